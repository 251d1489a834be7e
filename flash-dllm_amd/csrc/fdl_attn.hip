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
// Workgroup = one tile (up to 64*RB query rows of one sequence) x one head; eight
// wavefronts in two roles. Four producers move 64-key blocks of K and V from the cache
// (through the page table or key list) straight into LDS with global_load_lds, four
// blocks in flight; four consumers run the MFMAs and the online softmax from LDS and never
// issue a global load in the key loop. One workgroup barrier per block hands a block from
// producers to consumers and its buffer back.
//
// LDS layouts. K: key row of 256 B, 16-byte chunk c of key n at chunk c ^ (n & 15), read
// as the A operand of S^T = K Q^T (ds_read_b128, 16 consecutive keys on 16 distinct bank
// groups). V: key row of 256 B, chunk c at c ^ ((n & 7) << 1), read transposed as the A
// operand of O^T = V^T P^T with ds_read_b64_tr_b16: in each 16-lane group, source lane s
// reads 4 values V[n0 + s/4][d0 + 4 (s%4) ..] and output lane i receives
// V[n0 .. n0+3][d0 + i], i.e. four keys of one V^T row.
//
// Each consumer owns RB blocks of 16 query rows and computes S^T with 16x16x32 MFMAs, so
// lane l holds the logits of row l % 16 for keys 4*(l/16) + i of each 16-key block: the
// online-softmax max and sum need two cross-lane steps (xor 16, xor 32), and the bf16
// probabilities are already the B operand of O^T = V^T P^T. Importance needs column sums
// over rows instead, so it uses S = Q K^T (operand swap): 4 in-lane adds plus the same two
// cross-lane steps; the softmax-probability importance runs a second pass over K once the
// rows' log-sum-exp is known.
#include "fdl_device.h"
#include "fdl_host.h"

#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

namespace fdl {
namespace {

constexpr int kHeadDim = 128;
constexpr int kTileN = 64;                    // keys per block
constexpr int kProducers = 4;                 // producer wavefronts per workgroup
// LDS blocks in flight. Three stages, two of them loaded before the first block is handed
// over, measured faster than four (4-5% on 64-row tiles, 2% on Flash-Verify, results
// bit-identical): every CU starts by requesting its first stages at once, and the first
// block lands sooner the fewer requests are queued with it.
constexpr int kStages = 3;
constexpr int kFillStages = 2;  // stages loaded before the first block is handed over
constexpr int kTileBytes = kTileN * 256;      // one K (or V) block: 16 KB
constexpr int kStageBytes = 2 * kTileBytes;   // K then V
constexpr int kDmaPerTile = kTileBytes / 1024 / 4;  // 1 KB loads per producer per tile (4)
constexpr int kSlotCache = 2048;              // keys per workgroup whose slots are staged

typedef __attribute__((address_space(3))) void* lds_ptr;
typedef __attribute__((address_space(1))) void* glb_ptr;
typedef short s16x4 __attribute__((ext_vector_type(4)));

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
  const uint8_t* mask;       // verify: dense mask, or
  const int32_t* vmeta;      // verify: (T, S) per block, the closed-form mask
  float* imp_part;
  float* ws;         // softmax importance: probabilities of the importance rows (see kWsBlock)
  int ws_blocks;     // key blocks of room per (work item, head) in ws; 0: no workspace
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
  int split;         // 1: workgroup 2i + j runs rows [128 j, 128 j + 128) of 256-row item i
  int n_items;       // long tiles: work items of the launch (grid = n_items x heads)
  int head_groups;   // attn_kernel: groups of HPW heads; workgroup i runs head group
                     // i % head_groups of tile i / head_groups
  // key-split launches (no or raw importance): workgroup z of a (tile, head) takes the key
  // blocks [z nb / kv_parts, (z + 1) nb / kv_parts) and writes its unnormalised output and
  // (max, sum) per row into part_o (kPartFloats per (part, row-index entry, head));
  // attn_combine_kernel merges the parts
  float* part_o;
  int kv_parts;      // 1: no key split
};

// Record of one row's partial result: O (128 fp32, relative to the maximum), the maximum
// (log2 domain) and the sum, padded to a multiple of 4 floats.
constexpr int kPartFloats = 132;
constexpr int kMaxKvParts = 8;

template <int RB>
struct RowState {
  float m[RB];      // running max of the lane's rows (log2 domain)
  float l[RB];      // partial row sums
  f32x4 o[RB][8];   // O^T blocks: lane holds O[row][16*db + 4*(l/16) + i]
};

// Reductions over the four 16-lane rows of a wavefront (lane ^ 16, lane ^ 32) with gfx950's
// row-swap permutes, which run on the VALU and add no LDS traffic: permlane16_swap(x, x)
// returns {x of rows (0, 0, 2, 2), x of rows (1, 1, 3, 3)}, permlane32_swap(x, x) returns
// {rows (0, 1, 0, 1), rows (2, 3, 2, 3)}. The association matches a butterfly over xor 16
// then xor 32, so every lane gets the same bits.
__device__ __forceinline__ float xmax(float v) {
  const auto a =
      __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float m = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b =
      __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float xsum(float v) {
  const auto a =
      __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float m = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b =
      __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Sum over the 16 lanes of each lane group (lanes 16 g .. 16 g + 15) with DPP moves: quad
// exchanges (lane ^ 1, lane ^ 2), then the 8-lane and the 16-lane mirror; every step adds
// a lane pair in both orders, so all 16 lanes get the same bits.
__device__ __forceinline__ float dpp_add(float v, int ctrl_sel) {
  int t;
  switch (ctrl_sel) {
    case 0: t = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false); break;  // [1,0,3,2]
    case 1: t = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false); break;  // [2,3,0,1]
    case 2: t = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false); break;  // half mirror
    default: t = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false); break;  // mirror
  }
  return v + __int_as_float(t);
}
__device__ __forceinline__ float sum16(float v) {
  v = dpp_add(v, 0);
  v = dpp_add(v, 1);
  v = dpp_add(v, 2);
  return dpp_add(v, 3);
}

// Waits until at most n global loads of this wavefront are outstanding (n a multiple of
// 4 up to 16, the counts the producer pipeline can have).
__device__ __forceinline__ void wait_vmcnt(int n) {
  switch (n) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 8: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 12: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(16)" ::: "memory"); break;
  }
}
// Workgroup barrier without the compiler's memory fence (which would drain every
// outstanding global load); each role waits for exactly what it must first.
__device__ __forceinline__ void barrier_only() { asm volatile("s_barrier" ::: "memory"); }
__device__ __forceinline__ void barrier_lds_drained() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// K fragment (A operand of S^T = K Q^T): keys 16 kb + l16, d chunk 4 sd + g.
__device__ __forceinline__ bf16x8 k_frag(const u32x4* kt, int kb, int sd, int l16, int g) {
  return as_bf16x8(kt[(16 * kb + l16) * 16 + ((4 * sd + g) ^ l16)]);
}

// V^T fragment (A operand of O^T = V^T P^T) of PV step ks, d block db: k-slot (g, j) is key
// 32 ks + 4 g + j (j < 4) or 32 ks + 16 + 4 g + (j - 4); row d = 16 db + l16.
__device__ __forceinline__ bf16x8 vt_frag(const uint8_t* vt, int ks, int db, int l16, int g) {
  const int key = 32 * ks + 4 * g + (l16 >> 2);
  const int d = 16 * db + 4 * (l16 & 3);
  const int c = d >> 3, half = (d >> 2) & 1;
  const int off = ((c ^ ((key & 7) << 1)) << 4) + (half << 3);  // (key + 16) & 7 == key & 7
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(lds_ptr)(vt + key * 256 + off));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(lds_ptr)(vt + (key + 16) * 256 + off));
  u32x4 w;
  w[0] = __builtin_bit_cast(u32x2, lo)[0];
  w[1] = __builtin_bit_cast(u32x2, lo)[1];
  w[2] = __builtin_bit_cast(u32x2, hi)[0];
  w[3] = __builtin_bit_cast(u32x2, hi)[1];
  return as_bf16x8(w);
}

// Sum over the first n rows of a tile (row_idx[roff ..]) of Q[row][col], in ascending row
// order; 32 rows' index loads, then their Q loads, are in flight at a time.
__device__ __forceinline__ float sum_q_rows(const AttnArgs& a, int roff, int n, int64_t D,
                                           int col) {
  float acc = 0.f;
  for (int r0 = 0; r0 < n; r0 += 32) {
    int qr[32];
#pragma unroll
    for (int u = 0; u < 32; ++u) qr[u] = r0 + u < n ? a.row_idx[roff + r0 + u] : -1;
    float v[32];
#pragma unroll
    for (int u = 0; u < 32; ++u)
      v[u] = qr[u] >= 0 && qr[u] < a.n_q_rows ? bf2f(a.q[int64_t(qr[u]) * D + col]) : 0.f;
#pragma unroll
    for (int u = 0; u < 32; ++u)
      if (qr[u] >= 0 && qr[u] < a.n_q_rows) acc += v[u];
  }
  return acc;
}

// Raw importance is linear in Q: the column sums over the importance rows of Q K^T are
// (sum of those rows' Q) K^T. The fp32 sum x is split into three bf16 parts, hi = bf16(x),
// mid = bf16(x - hi), lo = bf16(x - hi - mid) (x - hi - mid - lo is below 2^-24 |x|), put in
// rows 0-2 of one 16-row MFMA A operand; the other rows are zero. Fragment sd covers head
// columns 32 sd .. 32 sd + 31: lane (l16, g) holds columns 32 sd + 8 g .. + 7 of row l16.
__device__ __forceinline__ u32x4 qsum_fragment(const float* qsum, int sd, int l16, int g) {
  u32x4 w = {0, 0, 0, 0};
  if (l16 < 3) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float x = qsum[32 * sd + 8 * g + 2 * j + e];
        const float hi = bf2f(f2bf(x));
        const float mid = bf2f(f2bf(x - hi));
        v[e] = l16 == 0 ? hi : l16 == 1 ? mid : x - hi - mid;
      }
      w[j] = pack_bf16x2(v[0], v[1]);
    }
  }
  return w;
}

// The dot product of the summed Q with a key from the MFMA result of qsum_fragment rows:
// lanes g == 0 hold rows 0-3 in acc[0..3]; the parts are added smallest first.
__device__ __forceinline__ float qsum_dot(const f32x4& acc) { return acc[0] + (acc[1] + acc[2]); }

// Running maxima are raised lazily: a row keeps its reference maximum until a block's
// logits exceed it by more than kLazyMax (log2 domain, a factor of 256), so the rescale of
// O and l is skipped for most blocks. Probabilities then stay below 256 (fp32 and bf16
// represent them to the same relative precision) and O / l is unchanged.
constexpr float kLazyMax = 8.f;

// One 64-key block of online softmax + PV for the wave's RB row blocks. bias(rb, kb, i) is
// 0 when row block rb's lane row may attend key 16*kb + 4*(l/16) + i of the block and
// -infinity when it may not; probs(rb, p, m) sees the block's fp32 probabilities of row
// block rb relative to the reference maximum m (log2 domain).
template <int RB, typename Bias, typename Probs>
__device__ __forceinline__ void attend_block(RowState<RB>& st, const bf16x8 (&qf)[RB][4],
                                             const u32x4* kt, const uint8_t* vt,
                                             float scale_log2, Bias bias, Probs probs) {
  const int lane = threadIdx.x & 63;
  const int l16 = lane & 15, g = lane >> 4;
  f32x4 sc[RB][4];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) sc[rb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
    for (int sd = 0; sd < 4; ++sd) {
      const bf16x8 kf = k_frag(kt, kb, sd, l16, g);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) sc[rb][kb] = mfma16(kf, qf[rb][sd], sc[rb][kb]);
    }
    // with two row blocks, keep the fragment reads of one 16-key block in flight at a time
    if constexpr (RB > 1) __builtin_amdgcn_sched_barrier(0);
  }
  float alpha[RB];
  bool rescale = false;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = __builtin_fmaf(sc[rb][kb][i], scale_log2, bias(rb, kb, i));
        sc[rb][kb][i] = v;
        tmax = fmaxf(tmax, v);
      }
    tmax = xmax(tmax);
    const bool raise = tmax > st.m[rb] + kLazyMax;
    const float m_new = raise ? tmax : st.m[rb];
    const float m_use = m_new == -INFINITY ? 0.f : m_new;  // nothing attended yet
    alpha[rb] = raise ? fast_exp2(st.m[rb] - m_use) : 1.f;
    rescale = rescale || raise;
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
    st.l[rb] = st.l[rb] * alpha[rb] + psum;
    probs(rb, sc[rb], m_use);  // p = 2^(logit - m_use) of the block, before the bf16 cast
  }
  if (__builtin_amdgcn_ballot_w64(rescale) != 0) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int db = 0; db < 8; ++db) st.o[rb][db] *= alpha[rb];
  }
  // k-slot (g, j) of PV step ks is key 32ks + 4g + j (j < 4) or 32ks + 16 + 4g + (j - 4)
  bf16x8 pb[RB][2];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pb[rb][ks][j] = static_cast<__bf16>(sc[rb][2 * ks][j]);
        pb[rb][ks][j + 4] = static_cast<__bf16>(sc[rb][2 * ks + 1][j]);
      }
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const bf16x8 vf = vt_frag(vt, ks, db, l16, g);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) st.o[rb][db] = mfma16(vf, pb[rb][ks], st.o[rb][db]);
    }
    if constexpr (RB > 1) __builtin_amdgcn_sched_barrier(0);
  }
}

// Column sums over the wave's importance rows of S = Q K^T for the 64 keys of a block:
// out[kb] (in every lane) = sum over rows of term(rb, i, s) for key 16*kb + (l % 16).
template <int RB, typename Term>
__device__ __forceinline__ void column_sums(float (&out)[4], const bf16x8 (&qf)[RB][4],
                                            const u32x4* kt, Term term) {
  const int lane = threadIdx.x & 63;
  const int l16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    f32x4 acc[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sd = 0; sd < 4; ++sd) {
      const bf16x8 kf = k_frag(kt, kb, sd, l16, g);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[rb] = mfma16(qf[rb][sd], kf, acc[rb]);  // S[4g+i][key]
    }
    float cs = 0.f;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i) cs += term(rb, i, acc[rb][i]);
    out[kb] = xsum(cs);
  }
}

// Softmax importance in one pass: the fp32 probabilities of up to kStoreRows importance rows
// are written, block by block, to the caller's workspace, each block relative to the row's
// reference maximum at that block, and the column sums are formed once the rows' log-sum-exp
// is known, so K is not read a second time. Per (work item, head) the workspace holds
// ws_blocks records of kWsBlock floats: [row][key] probabilities, then the rows' maxima.
constexpr int kStoreRows = 32;
constexpr int kWsBlock = kStoreRows * kTileN + kStoreRows;
// Up to kRegBlocks key blocks the probabilities stay on chip instead: the consumers hand each
// block's [row][key] probabilities to the producers through LDS (two buffers by block parity,
// rows padded to kPStride floats), and producer wave j % 4 keeps block j in registers, lane =
// key, all kStoreRows rows (32 registers per block); the rows' maxima stay in LDS.
constexpr int kRegBlocks = 24;
constexpr int kPStride = kTileN + 4;

// The Flash-Verify mask of a block of T fill rows, S draft rows and S mask rows (rows and
// columns in that order; generate.py:260-269): fill rows do not see the drafts; draft i sees
// drafts j <= i and masks j > i; mask i sees drafts j < i and masks j >= i; everything else
// is visible.
__device__ __forceinline__ bool verify_visible(int T, int S, int r, int j) {
  if (r < T) return j < T || j >= T + S;
  if (j < T) return true;
  const bool rd = r < T + S, cd = j < T + S;
  const int i = rd ? r - T : r - T - S, jj = cd ? j - T : j - T - S;
  if (rd) return cd ? i >= jj : i < jj;
  return cd ? i > jj : i <= jj;
}

// Steps of a tile, the same sequence for producers and consumers (one barrier each):
//   [0, n_blk)          cache blocks, K and V (verify: after the in-block keys)
//   [n_blk, 2 n_blk)    softmax importance without the LDS store: the cache blocks again,
//                       K only, last block first
//   verify (when the block has rows): the in-block keys first, in steps [0, n_ib) (they
//   were just written by the projection and come from L2 while the first cache blocks load)
// kSplit: a key-split launch (grid z = part; a.kv_parts > 1), a separate instance so that
// the unsplit kernels keep their code.
template <int RB, int NC, bool kVerify, int HPW = 1, bool kSplit = false>
__global__ __launch_bounds__(64 * (NC + kProducers), 1) void attn_kernel(AttnArgs a) {
  static_assert(HPW == 1 || (kVerify && HPW == 2), "several heads per workgroup: verify only");
  static_assert(!kSplit || (!kVerify && HPW == 1), "key split: block attention only");
  constexpr int kRows = 16 * RB * NC;
  constexpr int kSt = kStages;  // LDS ring depth
  __shared__ __align__(1024) uint8_t smem[kSt * kStageBytes];
  __shared__ float lse_buf[kRows];
  __shared__ int32_t slot_buf[kSlotCache];  // cache slot of key k_begin + i
  // Per importance mode (one per launch), in one union:
  union ImpLds {
    // raw: each consumer's column sums of its importance rows' Q, the summed Q as MFMA
    // A-operand fragments by lane, and the raw importance of key k_begin + i, written to
    // imp_part after the key loop (a consumer's global store inside the loop would wait
    // behind the producers' loads)
    struct {
      float qsum_part[kVerify ? 1 : NC][kHeadDim];
      u32x4 qsum_frag[kVerify ? 1 : 4][64];
      float raw[kVerify ? 1 : kSlotCache];
    } raw;
    // softmax importance, second pass over K: per-wave column sums of a block, by parity
    float cols[2][NC][kTileN];
    // softmax importance, probabilities on chip: a block's probabilities by parity, and
    // every block's row maxima (after the last block: the rows' factors 2^(m_j - lse))
    struct {
      float p[2][kStoreRows * kPStride];
      float m[kRegBlocks][kStoreRows];
    } reg;
  };
  __shared__ ImpLds imp_lds;
  auto& imp_buf = imp_lds.cols;
  auto& qsum_part = imp_lds.raw.qsum_part;
  auto& qsum_frag_buf = imp_lds.raw.qsum_frag;
  auto& raw_buf = imp_lds.raw.raw;

  const int tid = threadIdx.x;
  // The wavefront index is uniform; readfirstlane makes the role test a scalar branch, so a
  // wavefront executes only its own role's barriers (both roles execute 2 + HPW n_steps).
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const bool producer = wave >= NC;
  const int wr = producer ? wave - NC : wave;  // producer index or consumer index
  const int l16 = lane & 15, g = lane >> 4;
  // The grid is tile-major with the head group fastest, so workgroups start in work-list
  // order (longest tiles first) across all heads: a launch of several rounds ends with the
  // shortest tiles. Heads h .. h + HPW - 1, one after the other: the key steps of every
  // head run through the same LDS ring, so the next head's first blocks load while this
  // head finishes.
  const int tile = static_cast<int>(blockIdx.x / unsigned(a.head_groups));
  const int hg = static_cast<int>(blockIdx.x - unsigned(tile) * unsigned(a.head_groups));
  const int h = hg * HPW;
  const int64_t D = a.d_model;
  const int col0 = h * kHeadDim;

  int b = 0, k_begin, k_end, n_rows, n_imp = 0, row0 = 0, roff = 0;
  // verify: block vb_idx, rows [blk_row0 + 128 half, ...) of its n_in rows (all n_in rows
  // are also its in-block keys)
  int vb_idx = 0, half_v = 0, blk_row0 = 0, n_in = 0;
  if constexpr (kVerify) {
    vb_idx = a.split ? tile >> 1 : tile;
    half_v = a.split ? tile & 1 : 0;
    const int32_t* vb = a.vblocks + 4 * vb_idx;
    k_begin = vb[0];
    k_end = vb[1];
    blk_row0 = vb[2];
    n_in = vb[3] - vb[2];
    // out-of-range entries (rejected by the host validator) degrade to an empty range
    if (k_begin < 0 || k_end > a.n_keys) k_end = k_begin;
    if (blk_row0 < 0 || n_in < 0 || int64_t(blk_row0) + n_in > a.n_q_rows) n_in = 0;
    if (n_in > a.block_rows) n_in = a.block_rows;  // mask rows hold block_rows columns
    row0 = blk_row0 + kRows * half_v;
    n_rows = n_in - kRows * half_v;
    if (a.split && n_rows <= 0) return;  // an empty upper half
  } else {
    const int half = a.split ? tile & 1 : 0;
    const int32_t* it = a.work + 8 * (a.split ? tile >> 1 : tile);
    b = it[0];
    k_begin = it[1];
    k_end = it[2];
    roff = it[3] + 128 * half;
    n_rows = it[4] - 128 * half;
    n_imp = a.imp_mode && half == 0 ? it[5] : 0;
    if (b < 0 || b >= a.n_seq || k_begin < 0 ||
        int64_t(k_end) > (int64_t(a.max_pages) << a.page_log2)) {
      b = 0;
      k_end = k_begin;
    }
    if (roff < 0 || int64_t(roff) + (n_rows > 0 ? n_rows : 0) > a.n_row_idx) n_rows = 0;
  }
  if (n_rows > kRows) n_rows = kRows;
  if (n_rows < 0) n_rows = 0;
  if (!kVerify && n_rows == 0) return;  // the empty upper half of a split 128-row item
  if (n_imp > n_rows) n_imp = n_rows;
  if (k_end < k_begin) k_end = k_begin;
  if constexpr (kSplit) {
    // this workgroup's share of the tile's key blocks
    const int nb = (k_end - k_begin + kTileN - 1) / kTileN;
    const int z = static_cast<int>(blockIdx.z);
    const int j0 = z * nb / a.kv_parts, j1 = (z + 1) * nb / a.kv_parts;
    const int kb = k_begin;
    k_begin = kb + kTileN * j0;
    k_end = min(k_end, kb + kTileN * j1);
    if (k_end < k_begin) k_end = k_begin;
  }

  const bool imp_raw = !kVerify && n_imp > 0 && a.imp_mode == FDL_IMP_RAW_LOGIT;
  const bool imp_soft = !kVerify && n_imp > 0 && a.imp_mode == FDL_IMP_SOFTMAX_COLSUM;
  const int n_blk = (k_end - k_begin + kTileN - 1) / kTileN;
  const bool inblock = kVerify && n_rows > 0;
  const int n_ib = inblock ? (n_in + kTileN - 1) / kTileN : 0;  // in-block key steps
  // softmax importance in one pass with the probabilities on chip (up to kRegBlocks blocks)
  // or in the workspace, else from a second pass over K (64-row tiles only: the 128-row
  // variant's twelve wavefronts leave too few registers)
  const bool reg_store = NC == 4 && imp_soft && n_imp <= kStoreRows && n_blk <= kRegBlocks;
  const bool store =
      NC == 4 && imp_soft && !reg_store && n_imp <= kStoreRows && n_blk <= a.ws_blocks;
  const bool two_pass = imp_soft && !store && !reg_store;
  float* ws_tile = store ? a.ws + (int64_t(a.split ? tile >> 1 : tile) * a.head_groups + hg) *
                                   a.ws_blocks * kWsBlock
                         : nullptr;
  const int n_steps = n_blk * (two_pass ? 2 : 1) + n_ib;
  // Step -> key block: the first pass walks the blocks forward, the second (softmax
  // importance, K only) walks them backward, so it starts with the last kSt blocks of the
  // first pass, which are still in LDS, and continues with the most recently read ones.
  // Block j always lives in stage j % kSt; a resident block is not loaded again.
  auto block_of = [&](int step) {
    if constexpr (kVerify) return step - n_ib;
    return two_pass && step >= n_blk ? 2 * n_blk - 1 - step : step;
  };
  // Global step S = n_steps j + s: step s of head j. With several heads (verify: every step
  // a fresh block) step S lives in stage S % kSt.
  const int n_all = HPW * n_steps;
  auto stage_of = [&](int step) { return (HPW > 1 || kVerify ? step : block_of(step)) % kSt; };
  // DMA per producer for global step `step` (0: past the end, or a block still resident)
  auto loads = [&](int step) {
    if (step >= n_all) return 0;
    if (!kVerify && step >= n_blk) return step - n_blk < kSt ? 0 : kDmaPerTile;
    return 2 * kDmaPerTile;
  };
  // loads of steps (step, last] that may still be in flight once step `step` has landed
  auto later_loads = [&](int step, int last) {
    int n = 0;
    for (int t = step + 1; t <= last; ++t) n += loads(t);
    return n;
  };

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
  // The key -> slot map of the tile's key range is staged in LDS once, so the producers'
  // block loads do not wait on a page-table (or key-list) load first.
  const bool slots_staged = k_end - k_begin <= kSlotCache && n_slots < (int64_t(1) << 31);
  auto slot_of = [&](int n) -> int64_t {
    return slots_staged ? int64_t(slot_buf[n - k_begin]) : lookup(n);
  };

  float* imp_out = a.imp_part ? a.imp_part + int64_t(h) * n_slots : nullptr;
  if (producer) {
    const int tp = tid - 64 * NC;
    if (slots_staged) {
      for (int i = tp; i < k_end - k_begin; i += 256)
        slot_buf[i] = static_cast<int32_t>(lookup(k_begin + i));
    }
    barrier_lds_drained();  // #0: slot map staged
    // Load i of producer wr fills LDS bytes [1024 q, 1024 q + 1024) of a tile, q = 4 wr + i:
    // keys 4q .. 4q + 3; lane -> key 4q + lane / 16, LDS chunk lane % 16.
    const int pc = lane & 15;
    auto issue = [&](int gs) {
      if (loads(gs) == 0) return;
      uint8_t* st = smem + stage_of(gs) * kStageBytes;
      const int hj = HPW > 1 ? gs / n_steps : 0;  // head of the step
      const int s = gs - hj * n_steps;            // its step within the head
      const int colh = col0 + hj * kHeadDim;
      const bool in_blk = kVerify && s < n_ib;
      const bool k_only = !kVerify && s >= n_blk;
      const int n0 = k_begin + kTileN * block_of(s);
#pragma unroll
      for (int i = 0; i < kDmaPerTile; ++i) {
        const int q = kDmaPerTile * wr + i;
        const int key = 4 * q + (lane >> 4);
        const uint16_t *ks, *vs;
        if (in_blk) {
          // in-block key 64 s + key: query row blk_row0 + that (checked above)
          const int64_t r = int64_t(blk_row0) + min(kTileN * s + key, n_in - 1);
          ks = a.kblk + r * D + colh;
          vs = a.vblk + r * D + colh;
        } else {
          const int64_t slot = slot_of(min(n0 + key, k_end - 1));
          ks = a.k + slot * D + colh;
          vs = a.v + slot * D + colh;
        }
        const int kc = pc ^ (key & 15), vc = pc ^ ((key & 7) << 1);
        __builtin_amdgcn_global_load_lds((glb_ptr)(ks + 8 * kc), (lds_ptr)(st + 1024 * q), 16,
                                         0, 0);
        if (!k_only)
          __builtin_amdgcn_global_load_lds((glb_ptr)(vs + 8 * vc),
                                           (lds_ptr)(st + kTileBytes + 1024 * q), 16, 0, 0);
      }
    };
    static_assert(kFillStages >= 1 && kFillStages <= kSt, "fill");
    if (n_steps > 0) {
      for (int s = 0; s < kFillStages; ++s) issue(s);
      wait_vmcnt(later_loads(0, kFillStages - 1));  // step 0 landed
    }
    barrier_only();  // #1
    // the rest of the ring, while the consumers work on step 0
    for (int s = kFillStages; s < kSt; ++s) issue(s);
    // one step: wait for step s + 1, hand over step s, refill its stage
    auto step = [&](int s) {
      wait_vmcnt(later_loads(s + 1, s + kSt - 1));  // step s + 1 landed
      // consumers are done with step s (and this wave's reads of earlier probabilities)
      barrier_lds_drained();
      // step s + kSt lives in the stage of step s (a resident block's stage is kept)
      issue(s + kSt);
    };
    // on-chip softmax importance: producer wr keeps blocks j = wr, wr + 4, .. in pr[j / 4]
    // (rows 0 .. kStoreRows - 1 of key k_begin + 64 j + lane); the step loop is unrolled so
    // that every register index is static
    constexpr int kPrSlots = kVerify ? 1 : kRegBlocks / 4;
    float pr[kPrSlots][kVerify ? 1 : kStoreRows];
    if (!kVerify && reg_store) {
#pragma unroll
      for (int s = 0; s < kRegBlocks; ++s) {
        if (s < n_all) {
          step(s);
          if ((s & 3) == wr) {
            const float* src = imp_lds.reg.p[s & 1] + lane;
#pragma unroll
            for (int r = 0; r < kStoreRows; ++r) pr[(s >> 2) % kPrSlots][r] = src[r * kPStride];
          }
        }
      }
    } else {
      for (int s = 0; s < n_all; ++s) step(s);
    }
    wait_vmcnt(0);  // no load may still be writing LDS when the workgroup ends
    if constexpr (!kVerify) {
      if (reg_store) {
        // the last barrier made the last block's probabilities and the rows' factors
        // 2^(m_j - lse) visible; column sums over the importance rows in ascending row order
#pragma unroll
        for (int t = 0; t < kPrSlots; ++t) {
          const int j = 4 * t + wr;  // the block in pr[t]
          const int n = k_begin + kTileN * j + lane;
          if (j < n_blk && n < k_end) {
            // the factors of all rows first (uniform 16-byte reads), then the sums
            const f32x4* cv = reinterpret_cast<const f32x4*>(imp_lds.reg.m[j]);
            f32x4 c[kStoreRows / 4];
#pragma unroll
            for (int i = 0; i < kStoreRows / 4; ++i) c[i] = cv[i];
            float acc = 0.f;
#pragma unroll
            for (int r = 0; r < kStoreRows; ++r) acc = __builtin_fmaf(c[r / 4][r % 4], pr[t][r], acc);
            imp_out[slot_of(n)] = acc;
          }
        }
      }
    }
    if (store) __syncthreads();  // the consumers' workspace stores are complete
    return;
  }

  // ---------------------------------------------------------------- consumers
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
  }
  // the rows' Q columns of the head at column colh, and a fresh softmax state
  RowState<RB> st;
  auto load_q = [&](int colh, bf16x8 (&dst)[RB][4]) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int sd = 0; sd < 4; ++sd) {
        u32x4 v = {0, 0, 0, 0};
        if (qrow[rb] >= 0) v = ld16(a.q + qrow[rb] * D + colh + 32 * sd + 8 * g);
        dst[rb][sd] = as_bf16x8(v);
      }
  };
  auto reset_state = [&]() {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      st.m[rb] = -INFINITY;
      st.l[rb] = 0.f;
#pragma unroll
      for (int db = 0; db < 8; ++db) st.o[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  load_q(col0, qf);
  reset_state();
  // with several heads per workgroup the next head's Q columns load one head ahead, so the
  // consumers do not wait on them when the head changes
  bf16x8 qn[RB][4];
  if constexpr (HPW > 1) load_q(col0 + kHeadDim, qn);
  // verify: the block's (T, S) for the closed-form mask, read once
  int vT = 0, vS = 0;
  if (kVerify && a.vmeta) {
    vT = a.vmeta[2 * vb_idx];
    vS = a.vmeta[2 * vb_idx + 1];
  }
  const bool wave_imp = 16 * RB * wr < n_imp;
  const int imp_waves = (n_imp + 16 * RB - 1) / (16 * RB);
  float lse_r[RB][4];

  // Writes the importance sums of the block of step `s` (keys from n0): each consumer
  // wave sums 16 keys over the waves' partials. Runs after the barrier that follows the
  // partials' writes and before the barrier after which they are overwritten.
  auto flush_imp = [&](int s, int n0) {
    if (wr < 4 && l16 == lane) {  // lanes 0..15 of the first four consumers
      const int key = 16 * wr + lane;
      const int n = n0 + key;
      if (n < k_end) {
        float sum = 0.f;
        for (int w = 0; w < imp_waves; ++w) sum += imp_buf[s & 1][w][key];
        imp_out[slot_of(n)] = sum;
      }
    }
  };
  auto write_out = [&](int colh) {
    if constexpr (kSplit) {
      // a key split's part: the unnormalised row, its maximum and its sum
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        if (qrow[rb] < 0) continue;
        const int64_t ri = roff + 16 * (wr * RB + rb) + l16;
        float* rec = a.part_o + ((int64_t(blockIdx.z) * a.n_row_idx + ri) * a.head_groups + h) *
                                    kPartFloats;
#pragma unroll
        for (int db = 0; db < 8; ++db)
          *reinterpret_cast<f32x4*>(rec + 16 * db + 4 * g) = st.o[rb][db];
        if (g == 0) {
          rec[128] = st.m[rb];
          rec[129] = st.l[rb];
        }
      }
      return;
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      if (qrow[rb] < 0) continue;
      const float inv = st.l[rb] > 0.f ? 1.f / st.l[rb] : 0.f;
      uint16_t* orow = a.out + qrow[rb] * D + colh;
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        const f32x4 o = st.o[rb][db];
        const u32x2 pk = {pack_bf16x2(o[0] * inv, o[1] * inv),
                          pack_bf16x2(o[2] * inv, o[3] * inv)};
        st8(orow + 16 * db + 4 * g, pk);
      }
    }
  };

  // Raw importance from the summed Q (qsum_fragment): one wavefront per block computes all
  // 64 column sums. Each consumer first sums its importance rows' Q columns from its own Q
  // fragments (the 16 rows of a lane group, reduced across the group's lanes).
  if constexpr (!kVerify) {
    if (imp_raw && wave_imp) {
#pragma unroll
      for (int sd = 0; sd < 4; ++sd)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float v = 0.f;
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
            if (16 * (wr * RB + rb) + l16 < n_imp) v += static_cast<float>(qf[rb][sd][j]);
          v = sum16(v);
          if (l16 == 0) qsum_part[wr][32 * sd + 8 * g + j] = v;
        }
    }
  }
  barrier_lds_drained();  // #0
  // A-operand fragment sd of the summed Q (rows 0-2 its three bf16 parts), built by wave sd
  // from the consumers' partial sums, added in ascending consumer order
  if constexpr (!kVerify) {
    if (imp_raw && wr < 4) {
      float* qs = qsum_part[imp_waves - 1];
      if (lane < 32) {
        float v = 0.f;
        for (int w = 0; w < imp_waves; ++w) v += qsum_part[w][32 * wr + lane];
        qs[32 * wr + lane] = v;  // the last partial's own column, read only by wave wr
      }
      qsum_frag_buf[wr][lane] = qsum_fragment(qs, wr, l16, g);
    }
  }
  barrier_lds_drained();  // #1: step 0 landed; summed-Q fragments stored
  bool l_reduced = false;  // st.l holds per-lane partial sums until reduced across lanes
  for (int hj = 0; hj < HPW; ++hj) {
    if constexpr (HPW > 1) {
      if (hj > 0) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int sd = 0; sd < 4; ++sd) qf[rb][sd] = qn[rb][sd];
        if (hj + 1 < HPW) load_q(col0 + (hj + 1) * kHeadDim, qn);
        reset_state();
      }
    }
    for (int s = 0; s < n_steps; ++s) {
      const int stage = stage_of(hj * n_steps + s);
      const u32x4* kt = reinterpret_cast<const u32x4*>(smem + stage * kStageBytes);
      const uint8_t* vt = smem + stage * kStageBytes + kTileBytes;
      const bool pass2 = !kVerify && s >= n_blk;
      const bool in_blk = kVerify && s < n_ib;
      const int n0 = k_begin + kTileN * block_of(s);
      if (two_pass && s > n_blk) flush_imp(s - 1, k_begin + kTileN * block_of(s - 1));
      if (in_blk) {
        const int br = a.block_rows;
        const int j0 = kTileN * s;  // first in-block key of the step
        attend_block<RB>(st, qf, kt, vt, a.scale_log2, [&](int rb, int kb, int ii) {
          const int r = 16 * (wr * RB + rb) + l16;  // row of this workgroup
          const int rr = r + kRows * half_v;          // row of the block
          const int j = j0 + 16 * kb + 4 * g + ii;
          if (j >= n_in || r >= n_rows) return -INFINITY;
          const bool vis = a.vmeta ? verify_visible(vT, vS, rr, j)
                                   : a.mask[(int64_t(vb_idx) * br + rr) * br + j] != 0;
          return vis ? 0.f : -INFINITY;
        }, [](int, const f32x4 (&)[4], float) {});
      } else if (!pass2) {
        // keys past k_end (the tail of the last block) get a -infinity bias
        const int n_left = k_end - n0;
        float kbias[4][4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int ii = 0; ii < 4; ++ii)
            kbias[kb][ii] = 16 * kb + 4 * g + ii < n_left ? 0.f : -INFINITY;
        const int blk = block_of(s);
        attend_block<RB>(
            st, qf, kt, vt, a.scale_log2, [&](int, int kb, int ii) { return kbias[kb][ii]; },
            [&](int rb, const f32x4 (&p)[4], float m_use) {
              const int r = 16 * (wr * RB + rb) + l16;
              if (reg_store && r < kStoreRows) {
                // row r, keys 16 kb + 4 g .. + 3 of block blk, for producer blk % 4
                float* pr = imp_lds.reg.p[blk & 1] + r * kPStride;
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
                  *reinterpret_cast<f32x4*>(pr + 16 * kb + 4 * g) = p[kb];
                if (g == 0) imp_lds.reg.m[blk][r] = m_use;
              } else if (store && r < kStoreRows) {
                // row r, keys 16 kb + 4 g .. + 3 of block blk; then the row's maximum
                float* rec = ws_tile + int64_t(blk) * kWsBlock;
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
                  *reinterpret_cast<f32x4*>(rec + r * kTileN + 16 * kb + 4 * g) = p[kb];
                if (g == 0) rec[kStoreRows * kTileN + r] = m_use;
              }
            });
        if (imp_raw && wr < 4) {
          // consumer wr < 4: the 16 keys of key block kb = wr
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int sd = 0; sd < 4; ++sd)
            acc = mfma16(as_bf16x8(qsum_frag_buf[sd][lane]), k_frag(kt, wr, sd, l16, g), acc);
          const int n = n0 + 16 * wr + l16;
          if (g == 0 && n < k_end) {
            const float v = qsum_dot(acc);
            if constexpr (!kVerify) {
              if (slots_staged) raw_buf[n - k_begin] = v;
              else imp_out[slot_of(n)] = v;
            }
          }
        }
        if (imp_soft && s == n_blk - 1) {
          // end of the first pass: the rows' log2-sum-exp for the second pass
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) st.l[rb] = xsum(st.l[rb]);
          l_reduced = true;
          if (g == 0) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
              lse_buf[16 * (wr * RB + rb) + l16] =
                  st.l[rb] > 0.f ? st.m[rb] + log2f(st.l[rb]) : INFINITY;
          }
          if (reg_store) {
            // each block's row maximum becomes the row's factor 2^(m_j - lse), 0 for rows
            // past n_imp (lane group g takes blocks g, g + 4, ..), for the producers' column
            // sums after this step
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
              const int r = 16 * (wr * RB + rb) + l16;
              const float lse = st.l[rb] > 0.f ? st.m[rb] + log2f(st.l[rb]) : INFINITY;
              if (r < kStoreRows)
                for (int j = g; j < n_blk; j += 4)
                  imp_lds.reg.m[j][r] = r < n_imp ? fast_exp2(imp_lds.reg.m[j][r] - lse) : 0.f;
            }
          }
        }
      } else {
        if (s == n_blk) {
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) lse_r[rb][ii] = lse_buf[16 * (wr * RB + rb) + 4 * g + ii];
        }
        if (wave_imp) {
          float cs[4];
          column_sums<RB>(cs, qf, kt, [&](int rb, int ii, float sv) {
            return 16 * (wr * RB + rb) + 4 * g + ii < n_imp
                       ? fast_exp2(sv * a.scale_log2 - lse_r[rb][ii])
                       : 0.f;
          });
          if (g == 0) {
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) imp_buf[s & 1][wr][16 * kb + l16] = cs[kb];
          }
        }
      }
      barrier_lds_drained();  // step s consumed; step s + 1 landed
    }
    if (two_pass && n_steps > 0) flush_imp(n_steps - 1, k_begin + kTileN * block_of(n_steps - 1));
    // the output first: its accumulators are then free for the importance epilogue
    if (!l_reduced) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) st.l[rb] = xsum(st.l[rb]);
    }
    write_out(col0 + hj * kHeadDim);
  }
  if constexpr (!kVerify) {
    if (imp_raw && slots_staged) {
      // the last step's barrier made every block's sums visible
      for (int i = tid; i < k_end - k_begin; i += 64 * NC) imp_out[slot_buf[i]] = raw_buf[i];
    }
    if (NC == 4 && store) {
      // every block's probabilities and maxima are in the workspace once every consumer's
      // stores have completed (the barrier's release), the rows' log-sum-exp in LDS; column
      // sums over the importance rows in ascending row order
      wait_vmcnt(0);
      __syncthreads();
      const int nk = k_end - k_begin;
      for (int k0 = 4 * tid; k0 < nk; k0 += 4 * 64 * NC) {
        const int j = k0 / kTileN, u = k0 % kTileN;
        const float* rec = ws_tile + int64_t(j) * kWsBlock;
        // every row's probabilities and maximum are loaded before the first is used, so the
        // loads are in flight together (the callback above writes all kStoreRows rows of a
        // record, finite; rows past n_imp are dropped by the select)
        constexpr int kChunk = kStoreRows;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r0 = 0; r0 < kStoreRows; r0 += kChunk) {
          f32x4 pv[kChunk], mx[kChunk / 4];
#pragma unroll
          for (int i = 0; i < kChunk; ++i)
            pv[i] = *reinterpret_cast<const f32x4*>(rec + (r0 + i) * kTileN + u);
#pragma unroll
          for (int i4 = 0; i4 < kChunk / 4; ++i4)
            mx[i4] = *reinterpret_cast<const f32x4*>(rec + kStoreRows * kTileN + r0 + 4 * i4);
#pragma unroll
          for (int i = 0; i < kChunk; ++i) {
            const int r = r0 + i;
            const float c = fast_exp2(mx[i / 4][i % 4] - lse_buf[r]);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] = r < n_imp ? acc[e] + c * pv[i][e] : acc[e];
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int n = k_begin + k0 + e;
          if (n < k_end) imp_out[slot_of(n)] = acc[e];
        }
      }
    }
  }
}

// ------------------------------------------------------------------------------------------
// Long tiles (up to 256 query rows of one sequence x one head), for full recomputes.
//
// Eight wavefronts of 32 rows each in two groups, A (waves 0-3) and B (waves 4-7), one of
// each per SIMD. Every 64-key block j goes through an MFMA phase M_j (PV of block j-1, QK of
// block j) and a softmax phase V_j; group B runs one half-step behind group A, so in every
// half-step each SIMD has one wavefront issuing MFMAs and one running the softmax:
//   half-step 2j:     A: M_j                                B: V_{j-1}
//   half-step 2j + 1: A: V_j + the loads of block j + 2     B: M_j + transpose of V_j
// with a workgroup barrier between half-steps. Blocks move into a three-deep LDS ring (K and
// row-major V of a block, 32 KB). Every wavefront loads its share of the first three
// blocks; later blocks are loaded by group A alone, in its softmax phase (an MFMA phase
// would stall on the issue, and group B's softmax phase sits next to A's shorter MFMA
// phase). Each V block is rewritten once (block 0 by group A, later blocks by group B after
// its MFMA phase) into a fragment-major V^T buffer (two, by block parity) from which both
// groups read the O^T = V^T P^T operands with one 16-byte read per lane instead of two
// transposing reads.
//
// The loads are issued from inline assembly: the compiler then does not know them and
// inserts no wait for them before unrelated LDS reads; the waves wait for their own loads
// explicitly (s_waitcnt vmcnt) before the barrier that hands a block to the readers.
constexpr int kLongRows = 256;
constexpr int kLongStages = 3;
constexpr int kLongLoads = 4;  // 1 KB loads per wavefront per block (2 K + 2 V)

// 16 bytes per lane from global memory into LDS at lds + 16 * lane (lds wavefront-uniform).
// M0 carries the LDS address; its previous value is restored.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(lds)
      : "memory");
}

// Waits until at most n of this wavefront's global loads are outstanding (n = 0, 4, 8).
__device__ __forceinline__ void wait_loads(int n) {
  switch (n) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
  }
}

struct LongState {
  float m[2];
  float l[2];
  f32x4 o[2][8];
};

// Phase fences of the ping-pong. The barrier between a wavefront's MFMA phase and its
// softmax phase is an asm with a memory clobber, which orders memory operations only: the
// scheduler may move register-only work across it (it sank the exponentials, the bf16
// conversions and the row sums of a softmax phase into the next MFMA phase, next to the
// other group's softmax). settle(P) (an empty asm reading the probabilities) makes the
// softmax final before the barrier that ends its phase; hold(S) (one that "writes" the
// logits) keeps the softmax after the barrier that starts it. Both emit no instruction.
// (Fencing the MFMA results as well was measured 1-3% slower.)
__device__ __forceinline__ void hold(f32x4 (&v)[2][4]) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(v[i][j]));
}
__device__ __forceinline__ void settle(const bf16x8 (&v)[2][2]) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) asm volatile("" ::"v"(v[i][j]));
}

// V^T fragment i = 8 ks + db of the fragment-major buffer: one 16-byte read per lane.
__device__ __forceinline__ bf16x8 vtf_frag(const u32x4* vtf, int i, int lane) {
  return as_bf16x8(vtf[i * 64 + lane]);
}

// Rewrites fragments 4 wq .. 4 wq + 3 of a row-major V block as fragment-major V^T.
__device__ __forceinline__ void transpose_v(const uint8_t* vrow, u32x4* vtf, int wq, int lane) {
  const int l16 = lane & 15, g = lane >> 4;
  bf16x8 f[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = 4 * wq + j;
    f[j] = vt_frag(vrow, i >> 3, i & 7, l16, g);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) vtf[(4 * wq + j) * 64 + lane] = __builtin_bit_cast(u32x4, f[j]);
}

__device__ __forceinline__ void long_qk(f32x4 (&sc)[2][4], const bf16x8 (&qf)[2][4],
                                        const u32x4* kt, int l16, int g) {
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) sc[rb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int sd = 0; sd < 4; ++sd) {
      const bf16x8 kf = k_frag(kt, kb, sd, l16, g);
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) sc[rb][kb] = mfma16(kf, qf[rb][sd], sc[rb][kb]);
    }
}

__device__ __forceinline__ void long_pv(LongState& st, const bf16x8 (&pb)[2][2], const u32x4* vtf,
                                        int lane) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const bf16x8 vf = vtf_frag(vtf, i, lane);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) st.o[rb][i & 7] = mfma16(vf, pb[rb][i >> 3], st.o[rb][i & 7]);
  }
}

// M phase: PV of the previous block and QK of the current one in one schedule, the fragment
// reads three fragments ahead of the MFMAs that consume them. QK fragments go sd-major so
// consecutive MFMAs accumulate into different tiles.
__device__ __forceinline__ void long_pv_qk(LongState& st, const bf16x8 (&pb)[2][2],
                                           const u32x4* vtf, f32x4 (&sc)[2][4],
                                           const bf16x8 (&qf)[2][4], const u32x4* kt, int lane) {
  const int l16 = lane & 15, g = lane >> 4;
  bf16x8 vf[16], kf[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) vf[i] = vtf_frag(vtf, i, lane);
#pragma unroll
  for (int i = 0; i < 16; ++i) kf[i] = k_frag(kt, i & 3, i >> 2, l16, g);
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) st.o[rb][i & 7] = mfma16(vf[i], pb[rb][i >> 3], st.o[rb][i & 7]);
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) sc[rb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) sc[rb][i & 3] = mfma16(kf[i], qf[rb][i >> 2], sc[rb][i & 3]);
  __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);  // DS reads
#pragma unroll
  for (int i = 0; i < 29; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);
}

// V phase: online softmax of one block's logits (lane rows l % 16 of both row blocks), the
// lazily raised running maximum and the bf16 probabilities as PV operands. The maximum is
// taken over the raw logits and scaled once (the scale is positive), and each probability is
// 2^(fma(s, scale log2 e, -m)): one rounding and one VALU operation fewer per logit than
// scaling every logit first (3-4% on full recomputes). With kTail, keys
// 16 kb + 4 (l / 16) + i >= n_left are masked.
template <bool kTail>
__device__ __forceinline__ void long_softmax(LongState& st, f32x4 (&sc)[2][4], bf16x8 (&pb)[2][2],
                                             float scale_log2, int n_left, int g) {
  float alpha[2], mneg[2];
  bool rescale = false;
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (kTail)
          sc[rb][kb][i] = 16 * kb + 4 * g + i < n_left ? sc[rb][kb][i] : -INFINITY;
        tmax = fmaxf(tmax, sc[rb][kb][i]);
      }
    tmax = xmax(tmax) * scale_log2;
    const bool raise = tmax > st.m[rb] + kLazyMax;
    const float m_new = raise ? tmax : st.m[rb];
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    alpha[rb] = raise ? fast_exp2(st.m[rb] - m_use) : 1.f;
    rescale = rescale || raise;
    st.m[rb] = m_new;
    mneg[rb] = -m_use;
  }
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = fast_exp2(__builtin_fmaf(sc[rb][kb][i], scale_log2, mneg[rb]));
        sc[rb][kb][i] = p;
        psum += p;
      }
    st.l[rb] = st.l[rb] * alpha[rb] + psum;
  }
  if (__builtin_amdgcn_ballot_w64(rescale) != 0) {
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int db = 0; db < 8; ++db) st.o[rb][db] *= alpha[rb];
  }
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pb[rb][ks][j] = static_cast<__bf16>(sc[rb][2 * ks][j]);
        pb[rb][ks][j + 4] = static_cast<__bf16>(sc[rb][2 * ks + 1][j]);
      }
}

// Merges the kv_parts partial results of every row of a key-split launch: with m* the
// largest part maximum and w_p = 2^(m_p - m*) (0 for a part that attended nothing),
// out = (sum_p w_p O_p) / (sum_p w_p l_p), parts in ascending order, as bf16 like the
// unsplit kernel's rows. Grid = (work items, heads, tile rows / 8): thread t takes 4
// columns of one row; every part's values are loaded before the first is used.
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
  const int32_t* it = a.work + 8 * blockIdx.x;
  const int h = blockIdx.y;
  const int roff = it[3];
  int n_rows = it[4];
  if (roff < 0 || int64_t(roff) + (n_rows > 0 ? n_rows : 0) > a.n_row_idx) n_rows = 0;
  if (n_rows > a.tile_rows) n_rows = a.tile_rows;
  const int r = 8 * blockIdx.z + (threadIdx.x >> 5), c = 4 * (threadIdx.x & 31);
  if (r >= n_rows) return;
  const int64_t q = a.row_idx[roff + r];
  if (q < 0 || q >= a.n_q_rows) return;
  const int P = a.kv_parts;
  const int64_t stride = int64_t(a.n_row_idx) * gridDim.y * kPartFloats;  // between parts
  const float* rec0 = a.part_o + ((int64_t(roff) + r) * gridDim.y + h) * kPartFloats;
  float mp[kMaxKvParts], lp[kMaxKvParts];
  f32x4 op[kMaxKvParts];
#pragma unroll
  for (int p = 0; p < kMaxKvParts; ++p) {
    mp[p] = -INFINITY;
    lp[p] = 0.f;
    op[p] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (p < P) {
      const float* rec = rec0 + p * stride;
      mp[p] = rec[128];
      lp[p] = rec[129];
      op[p] = *reinterpret_cast<const f32x4*>(rec + c);
    }
  }
  float m = -INFINITY;
#pragma unroll
  for (int p = 0; p < kMaxKvParts; ++p) m = fmaxf(m, mp[p]);
  float l = 0.f;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int p = 0; p < kMaxKvParts; ++p) {
    const float w = mp[p] == -INFINITY ? 0.f : fast_exp2(mp[p] - m);
    l = __builtin_fmaf(w, lp[p], l);
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = __builtin_fmaf(w, op[p][e], o[e]);
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const u32x2 pk = {pack_bf16x2(o[0] * inv, o[1] * inv), pack_bf16x2(o[2] * inv, o[3] * inv)};
  st8(a.out + q * a.d_model + h * kHeadDim + c, pk);
}

// Importance: none or raw logits (the softmax-colsum mode runs the 128-row kernel on split
// items). Both groups execute 3 + 2 n_blk barriers.
__global__ __launch_bounds__(512, 1) void attn_long_kernel(AttnArgs a) {
  __shared__ __align__(1024) uint8_t smem[kLongStages * kStageBytes];
  __shared__ __align__(1024) u32x4 vtb[2][kTileBytes / 16];  // fragment-major V^T by parity
  __shared__ int32_t slot_buf[kSlotCache];
  __shared__ float qsum_buf[kHeadDim];
  __shared__ u32x4 qsum_frag_buf[4][64];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const bool grp_a = wave < 4;
  const int l16 = lane & 15, g = lane >> 4;
  // One-dimensional grid of items x heads. Workgroup i runs on XCD i % 8: renumber so that
  // each XCD gets a contiguous run of (head-major, item-minor) work, i.e. the tiles of one
  // sequence and head run on one XCD at about the same time and share its L2 for K and V.
  const int nwg = static_cast<int>(gridDim.x);
  int wid = static_cast<int>(blockIdx.x);
  if ((nwg & 7) == 0) wid = (wid & 7) * (nwg >> 3) + (wid >> 3);
  const int item = wid % a.n_items;
  const int h = wid / a.n_items;
  const int64_t D = a.d_model;
  const int col0 = h * kHeadDim;

  const int32_t* it = a.work + 8 * item;
  int b = it[0], k_begin = it[1], k_end = it[2], roff = it[3], n_rows = it[4];
  int n_imp = a.imp_mode ? it[5] : 0;
  if (b < 0 || b >= a.n_seq || k_begin < 0 ||
      int64_t(k_end) > (int64_t(a.max_pages) << a.page_log2)) {
    b = 0;
    k_end = k_begin;
  }
  if (roff < 0 || int64_t(roff) + (n_rows > 0 ? n_rows : 0) > a.n_row_idx) n_rows = 0;
  if (n_rows > kLongRows) n_rows = kLongRows;
  if (n_rows < 0) n_rows = 0;
  if (n_imp > n_rows) n_imp = n_rows;
  if (k_end < k_begin) k_end = k_begin;
  const bool imp_raw = n_imp > 0 && a.imp_mode == FDL_IMP_RAW_LOGIT;
  const int n_blk = (k_end - k_begin + kTileN - 1) / kTileN;

  const int pl = a.page_log2;
  const int pmask = (1 << pl) - 1;
  const int32_t* ptab = a.page_table + int64_t(b) * a.max_pages;
  const int64_t n_slots = a.n_slots;
  auto lookup = [&](int n) -> int64_t {
    const int64_t s = (int64_t(ptab[n >> pl]) << pl) | (n & pmask);
    return (s >= 0 && s < n_slots) ? s : 0;  // the host validators reject such tables
  };
  const bool slots_staged = k_end - k_begin <= kSlotCache && n_slots < (int64_t(1) << 31);
  auto slot_of = [&](int n) -> int64_t {
    return slots_staged ? int64_t(slot_buf[n - k_begin]) : lookup(n);
  };
  if (slots_staged) {
    for (int i = tid; i < k_end - k_begin; i += 64 * 8)
      slot_buf[i] = static_cast<int32_t>(lookup(k_begin + i));
  }

  // the wave's query rows: 32 wave + 16 rb + (lane % 16)
  int64_t qrow[2];
  bf16x8 qf[2][4];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int r = 32 * wave + 16 * rb + l16;
    qrow[rb] = -1;
    if (r < n_rows) {
      const int64_t q = int64_t(a.row_idx[roff + r]);
      if (q >= 0 && q < a.n_q_rows) qrow[rb] = q;
    }
#pragma unroll
    for (int sd = 0; sd < 4; ++sd) {
      u32x4 v = {0, 0, 0, 0};
      if (qrow[rb] >= 0) v = ld16(a.q + qrow[rb] * D + col0 + 32 * sd + 8 * g);
      qf[rb][sd] = as_bf16x8(v);
    }
  }
  if (imp_raw && tid < kHeadDim) qsum_buf[tid] = sum_q_rows(a, roff, n_imp, D, col0 + tid);
  __syncthreads();
  // raw importance: summed Q as three bf16 rows of one MFMA operand (see attn_kernel)
  if (imp_raw && wave < 4) qsum_frag_buf[wave][lane] = qsum_fragment(qsum_buf, wave, l16, g);
  // The Q loads are waited for here, before the first block load is issued: a later wait
  // the compiler places for them would also wait for every block load issued since.
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int sd = 0; sd < 4; ++sd) asm volatile("" ::"v"(qf[rb][sd]));
  __syncthreads();

  const uint32_t smem_lds = static_cast<uint32_t>(reinterpret_cast<size_t>((lds_ptr)smem));
  const int pc = lane & 15;
  // wave w loads keys 8 w .. 8 w + 7 of block blk: load i covers keys 8 w + 4 i + lane / 16
  // (1 KB of K, 1 KB of V), LDS chunk lane % 16 of each key row; keys past k_end repeat the
  // last key. The slots come from the staged slot map: a page-table read here is a vector
  // load, and the wait for it would also wait for every block load in flight (the ring's
  // look-ahead). Without a staged map, when the 8 keys share a page (k_begin % 8 == 0) their
  // slots come from one page-table entry.
  const bool scalar_pages = (k_begin & 7) == 0 && pl >= 3;
  const int64_t slot_last = n_blk > 0 ? lookup(k_end - 1) : 0;
  // the staged slots of the share of wavefront w (uniform) of block blk (LDS reads)
  auto staged_slots = [&](int blk, int w, int32_t (&sl)[2]) {
    const int n0 = k_begin + kTileN * blk;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      sl[i] = slot_buf[min(n0 + 8 * w + 4 * i + (lane >> 4), k_end - 1) - k_begin];
  };
  // the loads of that share, given its two slots
  auto issue_at = [&](int blk, int w, const int64_t (&slots)[2]) {
    const uint32_t st_lds = smem_lds + uint32_t((blk % kLongStages) * kStageBytes);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int q = 2 * w + i;
      const int key = 4 * q + (lane >> 4);
      const uint16_t* ks = a.k + slots[i] * D + col0;
      const uint16_t* vs = a.v + slots[i] * D + col0;
      const int kc = pc ^ (key & 15), vc = pc ^ ((key & 7) << 1);
      dma16(ks + 8 * kc, __builtin_amdgcn_readfirstlane(st_lds + 1024 * q));
      dma16(vs + 8 * vc, __builtin_amdgcn_readfirstlane(st_lds + kTileBytes + 1024 * q));
    }
  };
  auto issue = [&](int blk, int w) {
    const int n0 = k_begin + kTileN * blk;
    int64_t slots[2];
    if (slots_staged) {
      int32_t sl[2];
      staged_slots(blk, w, sl);
      slots[0] = sl[0];
      slots[1] = sl[1];
    } else if (scalar_pages) {
      const int nf = __builtin_amdgcn_readfirstlane(n0 + 8 * w);
      const int64_t base = nf < k_end ? int64_t(ptab[nf >> pl]) << pl : 0;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int n = nf + 4 * i + (lane >> 4);
        const int64_t s = base | (n & pmask);
        slots[i] = n < k_end && s >= 0 && s < n_slots ? s : slot_last;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i)
        slots[i] = slot_of(min(n0 + 8 * w + 4 * i + (lane >> 4), k_end - 1));
    }
    issue_at(blk, w, slots);
  };

  LongState st;
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    st.m[rb] = -INFINITY;
    st.l[rb] = 0.f;
#pragma unroll
    for (int db = 0; db < 8; ++db) st.o[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float* imp_out = a.imp_part ? a.imp_part + int64_t(h) * n_slots : nullptr;
  const float sl2 = a.scale_log2;
  auto kt_of = [&](int p) {
    return reinterpret_cast<const u32x4*>(smem + (p % kLongStages) * kStageBytes);
  };
  auto vt_of = [&](int p) -> const u32x4* { return vtb[p & 1]; };
  // V block p into the fragment-major V^T buffer of its parity, fragments 4 wq .. 4 wq + 3
  auto transpose = [&](int p, int wq) {
    transpose_v(smem + (p % kLongStages) * kStageBytes + kTileBytes, vtb[p & 1], wq, lane);
  };

  {
    // two blocks before the first hand-over, the third after it (a smaller first burst of
    // requests lands block 0 sooner: 1-2% on the stress batch's recomputes)
    const int np = min(n_blk, 2);
    for (int blk = 0; blk < np; ++blk) issue(blk, wave);
    if (np > 0) wait_loads(kLongLoads * (np - 1));  // block 0 landed
  }
  // Blocks past the first kLongStages are loaded by group A alone, both halves, in its
  // softmax phase (next to group B's MFMA phase, the longer one): group B's softmax phase
  // then holds no load issue, which stalls while the load queue is full.
  // At the end of pair p each wave waits for its loads of block p + 1 (block p + 2 may still
  // be in flight); the barrier that follows hands block p + 1 to all readers. Group A: one
  // share of block 1 (p = 0), both shares of later blocks; group B: only its shares of the
  // first kLongStages blocks.
  auto wait_next = [&](int p) {
    if (grp_a)
      wait_loads(p + 2 < n_blk ? (p == 0 ? kLongLoads : 2 * kLongLoads) : 0);
    else
      wait_loads(p == 0 && n_blk > 2 ? kLongLoads : 0);
  };
  barrier_only();
  if (n_blk > 2) issue(2, wave);  // the ring's third block, while block 0 is consumed
  if (n_blk > 0) {
    f32x4 sc[2][4];
    bf16x8 pb[2][2];
    if (grp_a) {
      auto run_a = [&](auto imp_tag) {
        constexpr bool kImp = decltype(imp_tag)::value;
        bf16x8 qs[4];
        if constexpr (kImp) {
#pragma unroll
          for (int sd = 0; sd < 4; ++sd) qs[sd] = as_bf16x8(qsum_frag_buf[sd][lane]);
        }
        // raw importance of block p: wave w sums keys 16 w .. 16 w + 15
        auto imp_block = [&](int p) {
          if constexpr (kImp) {
            const u32x4* kt = kt_of(p);
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int sd = 0; sd < 4; ++sd)
              acc = mfma16(qs[sd], k_frag(kt, wave, sd, l16, g), acc);
            const int n = k_begin + kTileN * p + 16 * wave + l16;
            if (g == 0 && n < k_end) imp_out[slot_of(n)] = qsum_dot(acc);
          }
        };
        long_qk(sc, qf, kt_of(0), l16, g);
        imp_block(0);
        barrier_only();
        if (n_blk == 1)
          long_softmax<true>(st, sc, pb, sl2, k_end - k_begin, g);
        else
          long_softmax<false>(st, sc, pb, sl2, kTileN, g);
        transpose(0, wave);
        if (n_blk > 1) wait_next(0);
        barrier_only();
        for (int p = 1; p < n_blk - 1; ++p) {
          // Block p + 2 goes into the stage of block p - 1, released in pair p - 1: one
          // share before the softmax, the other after it (each issue may wait for room in
          // the load queue). With a staged slot map its slots are read here, ahead of the
          // MFMA phase's fragment reads, so that the issues in the softmax phase wait for
          // no LDS read (1-3% faster).
          const bool ahead = slots_staged && p + 2 < n_blk;
          int32_t sa[2] = {0, 0}, sb[2] = {0, 0};
          if (ahead) {
            staged_slots(p + 2, wave, sa);
            staged_slots(p + 2, wave + 4, sb);
          }
          long_pv_qk(st, pb, vt_of(p - 1), sc, qf, kt_of(p), lane);
          imp_block(p);
          barrier_only();
          hold(sc);
          if (ahead)
            issue_at(p + 2, wave, {sa[0], sa[1]});
          else if (p + 2 < n_blk)
            issue(p + 2, wave);
          long_softmax<false>(st, sc, pb, sl2, kTileN, g);
          if (ahead)
            issue_at(p + 2, wave + 4, {sb[0], sb[1]});
          else if (p + 2 < n_blk)
            issue(p + 2, wave + 4);
          wait_next(p);
          settle(pb);
          barrier_only();
        }
        if (n_blk > 1) {
          const int p = n_blk - 1;
          long_pv_qk(st, pb, vt_of(p - 1), sc, qf, kt_of(p), lane);
          imp_block(p);
          barrier_only();
          long_softmax<true>(st, sc, pb, sl2, k_end - (k_begin + kTileN * p), g);
          barrier_only();
        }
        long_pv(st, pb, vt_of(n_blk - 1), lane);
        barrier_only();
        barrier_only();
      };
      if (imp_raw)
        run_a(std::true_type{});
      else
        run_a(std::false_type{});
    } else {
      barrier_only();
      long_qk(sc, qf, kt_of(0), l16, g);
      if (n_blk > 1) wait_next(0);
      barrier_only();
      for (int p = 1; p < n_blk; ++p) {
        hold(sc);
        long_softmax<false>(st, sc, pb, sl2, kTileN, g);
        settle(pb);
        barrier_only();
        long_pv_qk(st, pb, vt_of(p - 1), sc, qf, kt_of(p), lane);
        // V block p to V^T next to this MFMA phase (the other group's softmax phase then
        // holds only the softmax and the block loads)
        transpose(p, wave - 4);
        if (p + 1 < n_blk) wait_next(p);
        barrier_only();
      }
      long_softmax<true>(st, sc, pb, sl2, k_end - (k_begin + kTileN * (n_blk - 1)), g);
      barrier_only();
      long_pv(st, pb, vt_of(n_blk - 1), lane);
      barrier_only();
    }
  }
  wait_loads(0);  // no load may still be writing LDS when the workgroup ends
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    st.l[rb] = xsum(st.l[rb]);
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
    // one fma, as fdl_importance_accumulate_rank does for the step's last layer
    scores[s] = __builtin_fmaf(scale, sum, scores[s]);
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

// One workgroup per (tile, group of HPW heads), the head group fastest (see attn_kernel).
template <int RB, int NC, bool kVerify, int HPW = 1>
hipError_t launch_attn(AttnArgs args, int64_t n_tiles, int64_t n_heads, hipStream_t s) {
  const int64_t groups = n_heads / HPW;
  if (n_tiles * groups >= (int64_t(1) << 31)) return hipErrorInvalidValue;
  args.head_groups = static_cast<int>(groups);
  const dim3 grid(static_cast<unsigned>(n_tiles * groups));
  if constexpr (!kVerify) {
    if (args.kv_parts > 1) {
      hipLaunchKernelGGL((attn_kernel<RB, NC, false, 1, true>),
                         dim3(grid.x, 1, static_cast<unsigned>(args.kv_parts)),
                         dim3(64 * (NC + kProducers)), 0, s, args);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((attn_kernel<RB, NC, kVerify, HPW>), grid, dim3(64 * (NC + kProducers)), 0,
                     s, args);
  return hipGetLastError();
}

// Compute units of the current device (cached per device).
int attn_device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Flash-Verify launch: one workgroup per (block tile, head), one per CU at a time. A grid
// that would take more than one round of workgroups runs two heads per workgroup instead,
// so the second head's blocks stream in behind the first head's instead of paying a second
// round's start-up.
template <int RB, int NC>
hipError_t launch_verify(const AttnArgs& args, int64_t n_tiles, int64_t n_heads, hipStream_t s) {
  if (n_heads % 2 == 0 && n_tiles * n_heads > attn_device_cus())
    return launch_attn<RB, NC, true, 2>(args, n_tiles, n_heads, s);
  return launch_attn<RB, NC, true>(args, n_tiles, n_heads, s);
}

}  // namespace
}  // namespace fdl

namespace fdl {
namespace {

#define FDL_REQUIRE_ARG(p) FDL_REQUIRE((p) != nullptr, FDL_ERR_NULL, "%s: %s is NULL", fn, #p)

// Checks the arguments of a block-attention call and enqueues its kernels (the shared body
// of fdl_block_attention and fdl_block_attention_scores_noalloc).
int block_attention_launch(const char* fn, const void* q, const void* k_cache, const void* v_cache,
                           int64_t n_q_rows, int64_t n_slots, int64_t d_model, int64_t n_heads,
                           int64_t head_dim, const int32_t* page_table, int64_t n_seq,
                           int64_t max_pages, int32_t page_log2, const int32_t* work,
                           int64_t n_work, const int32_t* row_idx, int64_t n_row_idx,
                           int32_t tile_rows, float softmax_scale, void* out, int32_t imp_mode,
                           float* imp_part, float* workspace, int64_t workspace_floats,
                           hipStream_t s) {
  int rc = check_common(fn, q, k_cache, v_cache, out, d_model, n_heads, head_dim);
  if (rc != FDL_OK) return rc;
  FDL_REQUIRE_ARG(page_table);
  FDL_REQUIRE_ARG(work);
  FDL_REQUIRE_ARG(row_idx);
  FDL_REQUIRE(n_seq >= 1 && max_pages >= 1 && n_slots >= 1 && n_q_rows >= 1 && n_row_idx >= 1,
              FDL_ERR_SHAPE, "%s: empty table or cache", fn);
  FDL_REQUIRE(page_log2 >= 4 && page_log2 <= 12, FDL_ERR_SHAPE,
              "%s: page_log2 = %d outside [4, 12]", fn, page_log2);
  FDL_REQUIRE(max_pages << page_log2 < (int64_t(1) << 31) && n_seq < (int64_t(1) << 31),
              FDL_ERR_SHAPE, "%s: max_pages or n_seq too large", fn);
  FDL_REQUIRE(imp_mode >= FDL_IMP_NONE && imp_mode <= FDL_IMP_SOFTMAX_COLSUM, FDL_ERR_SHAPE,
              "%s: imp_mode = %d unknown", fn, imp_mode);
  FDL_REQUIRE(imp_mode == FDL_IMP_NONE || imp_part != nullptr, FDL_ERR_NULL,
              "%s: imp_part is NULL with imp_mode = %d", fn, imp_mode);
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
  FDL_REQUIRE(workspace_floats >= 0 && (workspace_floats == 0 || workspace != nullptr),
              FDL_ERR_NULL, "%s: workspace is NULL with workspace_floats = %lld", fn,
              (long long)workspace_floats);
  if (imp_mode == FDL_IMP_SOFTMAX_COLSUM && workspace != nullptr) {
    FDL_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, FDL_ERR_SHAPE,
                "%s: workspace must be 16-byte aligned", fn);
    // room per (work item, head), in key blocks (tiles beyond it take the second pass)
    const int64_t per = workspace_floats / (n_work * n_heads * kWsBlock);
    args.ws = workspace;
    args.ws_blocks = static_cast<int>(per < (int64_t(1) << 30) ? per : (int64_t(1) << 30));
  }
  args.n_slots = n_slots;
  args.n_q_rows = n_q_rows;
  args.max_pages = static_cast<int>(max_pages);
  args.page_log2 = page_log2;
  args.d_model = static_cast<int>(d_model);
  args.tile_rows = tile_rows;
  args.imp_mode = imp_mode;
  args.scale_log2 = softmax_scale * kLog2e;
  // Key split: a launch of 64- or 128-row tiles whose (tile, head) grid fills at most a
  // quarter of the device (without softmax-colsum importance, which needs every key of a
  // row) spreads each tile's key blocks over up to min(kMaxKvParts, CUs / grid) workgroups
  // (at least four fit; two parts on a half-filled device cost more than they save), as
  // many as the workspace holds partial rows for, then merges them. A caller that knows
  // the tiles' block counts gives room for no more parts than blocks, with the same result
  // bits: part z of p takes blocks [z nb / p, (z + 1) nb / p), so with p >= nb every
  // non-empty part is one block, empty parts merge as exact zeros, and one part is the
  // unsplit launch.
  int parts = 1;
  if (imp_mode != FDL_IMP_SOFTMAX_COLSUM && (tile_rows == 64 || tile_rows == 128) &&
      workspace != nullptr) {
    const int64_t cus = attn_device_cus(), grid = n_work * n_heads;
    if (4 * grid <= cus) {
      const int64_t room = workspace_floats / (n_row_idx * n_heads * kPartFloats);
      const int64_t p = std::min<int64_t>({kMaxKvParts, cus / grid, room});
      if (p >= 2) parts = static_cast<int>(p);
    }
  }
  if (parts > 1) {
    FDL_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, FDL_ERR_SHAPE,
                "%s: workspace must be 16-byte aligned", fn);
    args.part_o = workspace;
    args.kv_parts = parts;
  }
  // 64-row tiles: four consumers of 16 rows; 128-row tiles: eight consumers (two per SIMD);
  // 256-row tiles: the two-group kernel, or with softmax-colsum importance the 128-row
  // kernel on each half of an item (the importance rows lie in the first half)
  hipError_t e;
  if (tile_rows == 64) {
    e = launch_attn<1, 4, false>(args, n_work, n_heads, s);
  } else if (tile_rows == 128) {
    e = launch_attn<1, 8, false>(args, n_work, n_heads, s);
  } else if (imp_mode == FDL_IMP_SOFTMAX_COLSUM) {
    FDL_REQUIRE(n_work < (int64_t(1) << 30), FDL_ERR_SHAPE,
                "%s: n_work = %lld out of range", fn, (long long)n_work);
    args.split = 1;
    e = launch_attn<1, 8, false>(args, 2 * n_work, n_heads, s);
  } else {
    FDL_REQUIRE(n_work * n_heads < (int64_t(1) << 31), FDL_ERR_SHAPE,
                "%s: %lld items x %lld heads out of range", fn, (long long)n_work,
                (long long)n_heads);
    args.n_items = static_cast<int>(n_work);
    hipLaunchKernelGGL(attn_long_kernel, dim3(static_cast<unsigned>(n_work * n_heads)),
                       dim3(64 * 8), 0, s, args);
    e = hipGetLastError();
  }
  FDL_HIP_CHECK(e);
  if (parts > 1) {
    hipLaunchKernelGGL(attn_combine_kernel,
                       dim3(static_cast<unsigned>(n_work), static_cast<unsigned>(n_heads),
                            static_cast<unsigned>(tile_rows / 8)),
                       dim3(256), 0, s, args);
    FDL_HIP_CHECK(hipGetLastError());
  }
  return FDL_OK;
}

int importance_accumulate_launch(const char* fn, const float* imp_part, int64_t n_heads,
                                 int64_t n_slots, const int32_t* page_table, int64_t n_seq,
                                 int64_t max_pages, int32_t page_log2, const int32_t* work,
                                 int64_t n_work, float scale, float* scores, hipStream_t s) {
  FDL_REQUIRE(n_work >= 0 && n_work < 65536, FDL_ERR_SHAPE, "%s: n_work = %lld out of range", fn,
              (long long)n_work);
  if (n_work == 0) return FDL_OK;
  FDL_REQUIRE_ARG(imp_part);
  FDL_REQUIRE_ARG(page_table);
  FDL_REQUIRE_ARG(work);
  FDL_REQUIRE_ARG(scores);
  FDL_REQUIRE(n_heads >= 1 && n_slots >= 1 && n_seq >= 1 && max_pages >= 1, FDL_ERR_SHAPE,
              "%s: empty dimension", fn);
  FDL_REQUIRE(page_log2 >= 4 && page_log2 <= 12, FDL_ERR_SHAPE,
              "%s: page_log2 = %d outside [4, 12]", fn, page_log2);
  hipLaunchKernelGGL(imp_accumulate_kernel, dim3(4, static_cast<unsigned>(n_work)), dim3(256), 0,
                     s, imp_part, static_cast<int>(n_heads), n_slots, page_table,
                     static_cast<int>(n_seq), static_cast<int>(max_pages), page_log2, work, scale,
                     scores);
  FDL_HIP_CHECK(hipGetLastError());
  return FDL_OK;
}

// Library-owned device memory of fdl_block_attention_scores_noalloc: the per-head importance
// partials [n_heads][n_slots] (fp32). Every GPU the library runs on holds its own copy from
// module load until the process ends. In host code `scratch` names a host-side stand-in, not
// a device address: kernels get the address that hipGetSymbolAddress returns for the current
// device (scratch_on_current_device).
constexpr int64_t kScratchFloats = FDL_NOALLOC_SCRATCH_BYTES / 4;
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device, looked up once per device.
int scratch_on_current_device(float** ptr) {
  int dev = -1;
  FDL_HIP_CHECK(hipGetDevice(&dev));
  FDL_REQUIRE(dev >= 0 && dev < kMaxDevices, FDL_ERR_UNSUPPORTED,
              "fdl_block_attention_scores_noalloc: device %d beyond the %d supported", dev,
              kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    FDL_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    FDL_REQUIRE(p != nullptr, FDL_ERR_HIP,
                "fdl_block_attention_scores_noalloc: no device address for the scratch array");
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *ptr = g_scratch_ptr[dev];
  return FDL_OK;
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
                                   float* imp_part, float* workspace, int64_t workspace_floats,
                                   void* stream) {
  using namespace fdl;
  FDL_REQUIRE(n_work >= 0 && n_work < (int64_t(1) << 31), FDL_ERR_SHAPE,
              "fdl_block_attention: n_work = %lld out of range", (long long)n_work);
  FDL_REQUIRE(tile_rows == 64 || tile_rows == 128 || tile_rows == 256, FDL_ERR_UNSUPPORTED,
              "fdl_block_attention: tile_rows = %d (64, 128 or 256)", tile_rows);
  if (n_work == 0) return ok();
  const int rc = block_attention_launch("fdl_block_attention", q, k_cache, v_cache, n_q_rows, n_slots, d_model, n_heads,
                                        head_dim, page_table, n_seq, max_pages, page_log2, work,
                                        n_work, row_idx, n_row_idx, tile_rows, softmax_scale, out,
                                        imp_mode, imp_part, workspace, workspace_floats,
                                        static_cast<hipStream_t>(stream));
  return rc == FDL_OK ? ok() : rc;
}

extern "C" int fdl_block_attention_scores_noalloc(
    const void* q, const void* k_cache, const void* v_cache, int64_t n_q_rows, int64_t n_slots,
    int64_t d_model, int64_t n_heads, int64_t head_dim, const int32_t* page_table, int64_t n_seq,
    int64_t max_pages, int32_t page_log2, const int32_t* work, int64_t n_work,
    const int32_t* row_idx, int64_t n_row_idx, int32_t tile_rows, float softmax_scale, void* out,
    int32_t imp_mode, float imp_scale, float* scores, void* stream) {
  using namespace fdl;
  FDL_REQUIRE(n_work >= 0 && n_work < 65536, FDL_ERR_SHAPE,
              "fdl_block_attention_scores_noalloc: n_work = %lld out of range",
              (long long)n_work);
  FDL_REQUIRE(tile_rows == 64 || tile_rows == 128 || tile_rows == 256, FDL_ERR_UNSUPPORTED,
              "fdl_block_attention_scores_noalloc: tile_rows = %d (64, 128 or 256)", tile_rows);
  FDL_REQUIRE(imp_mode >= FDL_IMP_NONE && imp_mode <= FDL_IMP_SOFTMAX_COLSUM, FDL_ERR_SHAPE,
              "fdl_block_attention_scores_noalloc: imp_mode = %d unknown", imp_mode);
  FDL_REQUIRE(n_heads >= 1 && n_slots >= 1, FDL_ERR_SHAPE,
              "fdl_block_attention_scores_noalloc: empty dimension");
  FDL_REQUIRE(imp_mode == FDL_IMP_NONE || n_heads <= kScratchFloats / n_slots, FDL_ERR_UNSUPPORTED,
              "fdl_block_attention_scores_noalloc: %lld heads x %lld slots of importance "
              "partials exceed the %lld-byte scratch (FDL_NOALLOC_SCRATCH_BYTES)",
              (long long)n_heads, (long long)n_slots, (long long)FDL_NOALLOC_SCRATCH_BYTES);
  FDL_REQUIRE(imp_mode == FDL_IMP_NONE || scores != nullptr, FDL_ERR_NULL,
              "fdl_block_attention_scores_noalloc: scores is NULL with imp_mode = %d", imp_mode);
  if (n_work == 0) return ok();
  float* part = nullptr;
  if (imp_mode != FDL_IMP_NONE) {
    const int rc = scratch_on_current_device(&part);
    if (rc != FDL_OK) return rc;
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  // every partial the reduction reads is written by the attention first (the keys of the
  // importance tiles), so the scratch needs no clearing between calls
  // the scratch holds the partials [n_heads][n_slots], then (16-byte aligned) the softmax
  // importance workspace in what is left
  float* ws = nullptr;
  int64_t ws_floats = 0;
  if (imp_mode == FDL_IMP_SOFTMAX_COLSUM) {
    const int64_t off = (n_heads * n_slots + 3) / 4 * 4;
    ws = part + off;
    ws_floats = kScratchFloats - off;
  }
  int rc = block_attention_launch("fdl_block_attention_scores_noalloc", q, k_cache, v_cache,
                                  n_q_rows, n_slots, d_model, n_heads,
                                  head_dim, page_table, n_seq, max_pages, page_log2, work, n_work,
                                  row_idx, n_row_idx, tile_rows, softmax_scale, out, imp_mode,
                                  part, ws, ws_floats, s);
  if (rc == FDL_OK && imp_mode != FDL_IMP_NONE)
    rc = importance_accumulate_launch("fdl_block_attention_scores_noalloc", part, n_heads, n_slots, page_table, n_seq, max_pages,
                                      page_log2, work, n_work, imp_scale, scores, s);
  return rc == FDL_OK ? ok() : rc;
}

extern "C" int fdl_importance_accumulate(const float* imp_part, int64_t n_heads, int64_t n_slots,
                                         const int32_t* page_table, int64_t n_seq,
                                         int64_t max_pages, int32_t page_log2,
                                         const int32_t* work, int64_t n_work, float scale,
                                         float* scores, void* stream) {
  using namespace fdl;
  const int rc = importance_accumulate_launch("fdl_importance_accumulate", imp_part, n_heads,
                                              n_slots, page_table, n_seq,
                                              max_pages, page_log2, work, n_work, scale, scores,
                                              static_cast<hipStream_t>(stream));
  return rc == FDL_OK ? ok() : rc;
}

extern "C" int fdl_verify_attention(const void* q, const void* k_blk, const void* v_blk,
                                    const void* k_cache, const void* v_cache, int64_t n_q_rows,
                                    int64_t n_slots, int64_t d_model, int64_t n_heads,
                                    int64_t head_dim, const int64_t* key_slots, int64_t n_keys,
                                    const int32_t* vblocks, int64_t n_vblocks,
                                    const uint8_t* mask, const int32_t* vmeta,
                                    int32_t block_rows, float softmax_scale, void* out,
                                    void* stream) {
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
  FDL_REQUIRE((mask != nullptr) != (vmeta != nullptr), FDL_ERR_NULL,
              "fdl_verify_attention: exactly one of mask and vmeta must be given");
  FDL_REQUIRE((reinterpret_cast<uintptr_t>(k_blk) | reinterpret_cast<uintptr_t>(v_blk)) % 16 == 0,
              FDL_ERR_SHAPE, "fdl_verify_attention: k_blk/v_blk must be 16-byte aligned");
  FDL_REQUIRE(block_rows >= 1 && block_rows <= 256, FDL_ERR_UNSUPPORTED,
              "fdl_verify_attention: block_rows = %d outside [1, 256]", block_rows);
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
  args.vmeta = vmeta;
  args.block_rows = block_rows;
  args.n_slots = n_slots;
  args.n_q_rows = n_q_rows;
  args.n_keys = n_keys;
  args.d_model = static_cast<int>(d_model);
  args.scale_log2 = softmax_scale * kLog2e;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  // up to 64 rows per block: 64-row tiles; up to 128: 128-row tiles; up to 256: two 128-row
  // workgroups per block (each attends to every in-block key)
  hipError_t e;
  if (block_rows <= 64) {
    e = launch_verify<1, 4>(args, n_vblocks, n_heads, s);
  } else {
    FDL_REQUIRE(n_vblocks < (int64_t(1) << 30), FDL_ERR_SHAPE,
                "fdl_verify_attention: n_vblocks out of range");
    args.split = block_rows > 128 ? 1 : 0;
    e = launch_verify<1, 8>(args, block_rows > 128 ? 2 * n_vblocks : n_vblocks, n_heads, s);
  }
  FDL_HIP_CHECK(e);
  return ok();
}
