// Fused QKV projection + rotate-half RoPE + direct K/V cache write (gfx950, bf16 MFMA).
//
// Follows _flash_qkv_proj_cache_fwd (flash_cache_triton.py:15-100) and
// _flash_verify_qkv_proj_fwd (flash_cache_triton.py:255-338):
//   q~ = x_r W_q^T, k~ = x_r W_k^T, v~ = x_r W_v^T           (fp32 accumulation)
//   Q[r, h*128 + c]      = q~_c cos[s, c]      - q~_{c+64} sin[s, c]
//   Q[r, h*128 + c + 64] = q~_{c+64} cos[s, c+64] + q~_c sin[s, c+64]       (c < 64)
//   K is rotated the same way; V is not rotated.
//   Q goes to packed row r; K/V go to cache row slot[r] (or packed row r for verify).
//
// The output columns are handled as RoPE pairs (c, c + 64) of a head: pair p of the
// 3 * n_heads * 64 pairs is column c = p % 64 of head (p / 64) % n_heads of matrix
// p / (64 * n_heads). A tile is a block of rows times a block of pairs, and a wavefront
// computes both members of its pairs, so lane l holds (c, c + 64) of the same rows in the
// same accumulator slot and RoPE runs in registers before the bf16 stores.
//
// One kernel, qkv_pc_kernel<BM, BP, NPROD, STAGES>: a workgroup computes BM rows x BP pairs
// with wavefronts in two roles. NPROD producers move the X and W tiles of each 64-wide
// reduction step straight from global memory into LDS (global_load_lds), STAGES steps deep;
// four consumers (one per SIMD, a 2 x 2 grid over rows and pairs) run the 16x16x32 MFMAs
// from LDS. A consumer never issues a global memory instruction, so its MFMA stream is
// never held behind the texture-address queue. After the reduction the consumers stage the
// fp32 sums in the (then free) stage memory and every wavefront rotates and writes 8-pair
// groups with 16-byte stores. Two shapes, chosen by the number of rows:
//  * more than 128 rows: 128 rows x 96 pairs, 4 stages of 40 KB (all of LDS). 512 rows give
//    one tile per CU.
//  * up to 128 rows (weight streaming, HBM-bound): 64 or 128 rows x 32 pairs (192 tiles at
//    d_model 4096), 8 stages of 16 KB or 6 of 24 KB, so each workgroup keeps 5-7 weight
//    steps in flight.
#include <atomic>
#include <type_traits>

#include "fdl_device.h"
#include "fdl_host.h"

namespace fdl {
namespace {

constexpr int kHeadDim = 128;
constexpr int kHalf = 64;
constexpr int kKT = 64;  // reduction step, bf16 elements (8 chunks of 16 B per row)
constexpr int kDAlign = 256;  // d_model must be a multiple of this

struct QkvArgs {
  const uint16_t* x;
  const uint16_t* w[3];
  const float* sin;
  const float* cos;
  const int64_t* slot;
  const int64_t* rope_row;
  uint16_t* q_out;
  uint16_t* k_out;
  uint16_t* v_out;
  int64_t n_rows;
  int64_t n_rope_rows;
  int64_t n_kv_rows;
  int d_model;
  int n_heads;
  int n_mtiles;
  int n_tiles;
  int kv_packed;
  int rope_half;  // sin/cos rows repeat their first half: read only that half
};

// LDS tile layout: chunk c (16 B) of tile row r is stored at chunk c ^ ((r >> 1) & 7) of
// that row: two 128-byte rows share one 256-byte bank line, so 16 consecutive rows read at
// the same logical chunk land on 16 distinct 4-bank groups.

// Workgroup i runs on XCD i % 8. Renumber so that each XCD gets a contiguous run of tiles
// (tiles are numbered n-block-major): the m-tiles that share one weight slice then run on
// one XCD and share its L2.
__device__ __forceinline__ int xcd_tile(int bid, int n_tiles) {
  return (n_tiles & 7) == 0 ? (bid & 7) * (n_tiles >> 3) + (bid >> 3) : bid;
}

// Tile t -> (n-block, m-block). Tiles come in groups of kGroupM m-blocks: within a group
// the m-block varies fastest, so the tiles running at the same time on one XCD share both
// X row blocks (kGroupM of them) and weight slices (one per kGroupM tiles) in its L2.
// With at most kGroupM m-blocks this is the plain n-block-major order.
constexpr int kGroupM = 8;
__device__ __forceinline__ void tile_coords(int t, int n_mtiles, int n_tiles, int& nt, int& mt) {
  const int n_ntiles = n_tiles / n_mtiles;
  const int per_group = kGroupM * n_ntiles;
  const int grp = t / per_group, r = t - grp * per_group;
  const int gm = min(kGroupM, n_mtiles - grp * kGroupM);  // m-blocks in this group
  nt = r / gm;
  mt = grp * kGroupM + (r - nt * gm);
}

// Destinations of row r: dq = Q row, dkv = K/V row (cache slot, or the packed row), rope =
// sin/cos row. A row past n_rows, or with an out-of-range slot or rope row, gets -1 in all
// three (skipped in all three outputs).
__device__ __forceinline__ void row_dest(const QkvArgs& a, int64_t r, int64_t& dq, int64_t& dkv,
                                         int64_t& rope) {
  dq = dkv = rope = -1;
  if (r < a.n_rows) {
    const int64_t s = a.slot[r];
    const int64_t rr = a.rope_row ? a.rope_row[r] : s;
    const bool rope_ok = rr >= 0 && rr < a.n_rope_rows;
    const bool slot_ok = a.kv_packed || (s >= 0 && s < a.n_kv_rows);
    if (rope_ok && slot_ok) {
      dq = r;
      dkv = a.kv_packed ? r : s;
      rope = rr;
    }
  }
}

// 8 consecutive pairs (c0 .. c0 + 7 of one head; lo = q~_c, hi = q~_{c+64}) of one row:
// load() reads the fp32 sums from LDS and the sin/cos values, store() rotates and writes two
// 16-byte bf16 chunks. c0 is a multiple of 8, so the sin/cos reads and both stores are
// 16-byte aligned. A group whose row has no destination (dst < 0) reads and writes nothing.
struct EpGroup {
  f32x4 lo[2], hi[2];
  f32x4 s1[2], s2[2], c1[2], c2[2];
  int64_t dst;
  int mat, head, c0;

  __device__ __forceinline__ void load(const QkvArgs& a, const float* src, int hi_off, int m,
                                       int rem, int64_t d, int64_t rope) {
    mat = m;
    head = rem >> 6;
    c0 = rem & 63;
    dst = d;
    if (d < 0) return;
    lo[0] = *reinterpret_cast<const f32x4*>(src);
    lo[1] = *reinterpret_cast<const f32x4*>(src + 4);
    hi[0] = *reinterpret_cast<const f32x4*>(src + hi_off);
    hi[1] = *reinterpret_cast<const f32x4*>(src + hi_off + 4);
    if (m < 2) {
      const float* sn = a.sin + rope * kHeadDim + c0;
      const float* cs = a.cos + rope * kHeadDim + c0;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        s1[h] = *reinterpret_cast<const f32x4*>(sn + 4 * h);
        c1[h] = *reinterpret_cast<const f32x4*>(cs + 4 * h);
        if (a.rope_half) {
          s2[h] = s1[h];
          c2[h] = c1[h];
        } else {
          s2[h] = *reinterpret_cast<const f32x4*>(sn + kHalf + 4 * h);
          c2[h] = *reinterpret_cast<const f32x4*>(cs + kHalf + 4 * h);
        }
      }
    }
  }

  __device__ __forceinline__ void store(const QkvArgs& a) {
    if (dst < 0) return;
    float l[8], r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      l[j] = lo[j >> 2][j & 3];
      r[j] = hi[j >> 2][j & 3];
    }
    if (mat < 2) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int h = j >> 2, e = j & 3;
        const float rlo = l[j] * c1[h][e] - r[j] * s1[h][e];
        const float rhi = r[j] * c2[h][e] + l[j] * s2[h][e];
        l[j] = rlo;
        r[j] = rhi;
      }
    }
    const u32x4 wlo = {pack_bf16x2(l[0], l[1]), pack_bf16x2(l[2], l[3]), pack_bf16x2(l[4], l[5]),
                       pack_bf16x2(l[6], l[7])};
    const u32x4 whi = {pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3]), pack_bf16x2(r[4], r[5]),
                       pack_bf16x2(r[6], r[7])};
    uint16_t* base = mat == 0 ? a.q_out : (mat == 1 ? a.k_out : a.v_out);
    uint16_t* d = base + dst * a.d_model + int64_t(head) * kHeadDim + c0;
    // non-temporal: the whole grid writes its Q/K/V rows at once at the end (1.5% faster at
    // 512 rows, 2% at 6842; the attention that reads them next is unchanged)
    __builtin_nontemporal_store(wlo, reinterpret_cast<u32x4*>(d));
    __builtin_nontemporal_store(whi, reinterpret_cast<u32x4*>(d + kHalf));
  }
};

typedef __attribute__((address_space(3))) void* lds_ptr;
typedef __attribute__((address_space(1))) void* glb_ptr;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Waits until at most n (clamped to 0 .. STAGES - 1) steps of kLoads loads each are in flight.
template <int STAGES, int kLoads>
__device__ __forceinline__ void wait_steps(int n) {
  static_assert(STAGES >= 2 && STAGES <= 8, "stages");
  switch (n <= 0 ? 0 : (n >= STAGES - 1 ? STAGES - 1 : n)) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<kLoads>(); break;
    case 2: wait_vmcnt<(STAGES > 2 ? 2 : 0) * kLoads>(); break;
    case 3: wait_vmcnt<(STAGES > 3 ? 3 : 0) * kLoads>(); break;
    case 4: wait_vmcnt<(STAGES > 4 ? 4 : 0) * kLoads>(); break;
    case 5: wait_vmcnt<(STAGES > 5 ? 5 : 0) * kLoads>(); break;
    case 6: wait_vmcnt<(STAGES > 6 ? 6 : 0) * kLoads>(); break;
    default: wait_vmcnt<(STAGES > 7 ? 7 : 0) * kLoads>(); break;
  }
}
// Workgroup barrier without the compiler's memory fence; each side waits for exactly the
// memory operations it must (the fence would drain every outstanding global load).
__device__ __forceinline__ void barrier_lds_drained() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
__device__ __forceinline__ void barrier_only() { asm volatile("s_barrier" ::: "memory"); }

// ---------------------------------------------------------------------------------------
// Shape of one qkv_pc_kernel instance. Consumer (wm, wn), wm, wn < 2, owns rows
// BM/2 * wm .. + BM/2 and pairs BP/2 * wn .. + BP/2 (low and high columns).
template <int BM, int BP, int NPROD, int STAGES>
struct PcShape {
  static constexpr int kConsumers = 4;
  static constexpr int kThreads = (kConsumers + NPROD) * 64;
  static constexpr int kWP = BP / 2, kPB = kWP / 16, kRB = BM / 32;
  static constexpr int kABytes = BM * 128;                 // X tile of one step
  static constexpr int kStageBytes = kABytes + 2 * BP * 128;  // + W tile (low, high columns)
  static constexpr int kLoads = kStageBytes / 1024 / NPROD;   // 1 KB loads per producer/step
  // Epilogue staging in the stage memory once the reduction is done: the fp32 sums as rows
  // of [BP low | BP high] columns (row stride padded by 4 floats), then the rows'
  // destinations (Q row, K/V row, sin/cos row).
  static constexpr int kEpStride = 2 * BP + 4;
  static constexpr int kEpMetaOff = BM * kEpStride * 4;
  static_assert(kPB >= 1 && kRB >= 1 && kPB * 16 == kWP && kRB * 32 == BM, "tile shape");
  static_assert(kLoads * NPROD * 1024 == kStageBytes, "producer split");
  static_assert((STAGES - 1) * kLoads < 64, "vmcnt range");
  static_assert(STAGES * kStageBytes <= 160 * 1024, "LDS");
  static_assert(kEpMetaOff + 3 * BM * 8 <= STAGES * kStageBytes, "epilogue staging");
  static_assert(BM <= kThreads, "row destinations");
};

template <int BM, int BP, int NPROD, int STAGES>
__global__ __launch_bounds__((4 + NPROD) * 64, 1) void qkv_pc_kernel(QkvArgs a) {
  using Sh = PcShape<BM, BP, NPROD, STAGES>;
  constexpr int kWP = Sh::kWP, kPB = Sh::kPB, kRB = Sh::kRB, kLoads = Sh::kLoads;
  constexpr int kStageBytes = Sh::kStageBytes, kEpStride = Sh::kEpStride;
  constexpr int kThreads = Sh::kThreads, kConsumers = Sh::kConsumers;
  __shared__ __align__(1024) uint8_t smem[STAGES * kStageBytes];

  const int tid = threadIdx.x;
  int nt, mt;
  tile_coords(xcd_tile(blockIdx.x, a.n_tiles), a.n_mtiles, a.n_tiles, nt, mt);
  const int64_t m0 = int64_t(mt) * BM;
  const int D = a.d_model;
  const int pairs_per_mat = a.n_heads * kHalf;
  // The wavefront index is uniform; readfirstlane makes the role test a scalar branch, so a
  // wavefront executes only its own role's barriers (both roles execute 3 + nk of them).
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const bool producer = wave >= kConsumers;
  const int nk = D / kKT;

  // Destinations of tile rows 0 .. BM - 1 (threads 0 .. BM - 1), read now and staged in LDS
  // for the epilogue once the stage memory is free.
  int64_t my_dq = -1, my_dkv = -1, my_rope = -1;
  if (tid < BM) row_dest(a, m0 + tid, my_dq, my_dkv, my_rope);

  if (producer) {
    const int pw = wave - kConsumers;
    // Load i of producer pw fills LDS bytes [1024 q, 1024 q + 1024) of the step's tile
    // (q = NPROD i + pw, an 8-row block): lane -> row 8 q + lane / 8, LDS chunk lane % 8,
    // which holds the row's logical chunk (lane % 8) ^ ((row >> 1) & 7) (the LDS tile
    // layout). Tile rows past n_rows re-read row n_rows - 1 (never stored). The blocks are
    // dealt round-robin, so every producer requests both X and weight rows: with the X rows
    // on some producers and the weights on the others, the 40-row projection took 2% longer.
    const uint16_t* src[kLoads];
    int dst_off[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int q = NPROD * i + pw;
      const int row = 8 * q + (lane >> 3);
      const int c = (lane & 7) ^ ((row >> 1) & 7);
      if (row < BM) {
        src[i] = a.x + min(m0 + row, a.n_rows - 1) * D + 8 * c;
      } else {
        const int wr = row - BM, hlf = wr / BP;
        const int p = BP * nt + (wr - hlf * BP);
        const int mat = p / pairs_per_mat, rem = p - mat * pairs_per_mat;
        src[i] = a.w[mat] + int64_t((rem >> 6) * kHeadDim + (rem & 63) + kHalf * hlf) * D +
                 8 * c;
      }
      dst_off[i] = 1024 * q;
    }
    // Requests step kt (< nk) into `stage`. No step past the end is requested: the tail of the
    // loop waits for fewer steps instead (re-reading the last step there, to keep one wait
    // count, cost 1.3% at 512 rows).
    auto issue = [&](int kt, int stage) {
      const int k0 = kt * kKT;
      uint8_t* st = smem + stage * kStageBytes;
#pragma unroll
      for (int i = 0; i < kLoads; ++i)
        __builtin_amdgcn_global_load_lds((glb_ptr)(src[i] + k0), (lds_ptr)(st + dst_off[i]), 16,
                                         0, 0);
    };
    const int first = min(STAGES, nk);  // steps requested before the loop
#pragma unroll
    for (int s = 0; s < STAGES; ++s)
      if (s < first) issue(s, s);
    wait_steps<STAGES, kLoads>(first - 1);  // step 0 landed
    barrier_only();
    int stage = 0;
    int kt = 0;
    for (; kt + STAGES < nk; ++kt) {
      // step kt + 1 landed (steps kt + 2 .. kt + STAGES - 1 may still be in flight)
      wait_vmcnt<(STAGES - 2) * kLoads>();
      barrier_only();
      issue(kt + STAGES, stage);  // this stage's last reads came before the barrier
      stage = stage == STAGES - 1 ? 0 : stage + 1;
    }
    // the last steps request nothing: step kt + 1 landed, steps kt + 2 .. nk - 1 in flight
    for (; kt < nk; ++kt) {
      wait_steps<STAGES, kLoads>(nk - 2 - kt);
      barrier_only();
    }
    wait_vmcnt<0>();  // no load may still be writing LDS when the stages are reused
    barrier_only();   // -> the consumers may overwrite the stages
    barrier_only();   // <- the accumulators and destinations are staged
  } else {
    const int wm = wave >> 1, wn = wave & 1;  // rows BM/2 wm .., pairs BP/2 wn ..
    const int l16 = lane & 15, g4 = lane >> 4;
    const int sw = (l16 >> 1) & 7;
    struct Frag {
      u32x4 a[kRB];
      u32x4 b[2][kPB];
    };
    // MFMA operands of half-step ss of the step in `stage`: lane (l16, g4) takes logical
    // chunk 4 ss + g4 of its row.
    auto read_frag = [&](Frag& f, int stage, int ss) {
      const u32x4* st = reinterpret_cast<const u32x4*>(smem + stage * kStageBytes);
      const int c = (4 * ss + g4) ^ sw;
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) f.a[rb] = st[((BM / 2) * wm + 16 * rb + l16) * 8 + c];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int pb = 0; pb < kPB; ++pb)
          f.b[h][pb] = st[Sh::kABytes / 16 + (BP * h + kWP * wn + 16 * pb + l16) * 8 + c];
    };
    f32x4 acc[kRB][2][kPB];
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int pb = 0; pb < kPB; ++pb) acc[rb][h][pb] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto mma = [&](const Frag& f) {
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int pb = 0; pb < kPB; ++pb)
            acc[rb][h][pb] = mfma16(as_bf16x8(f.a[rb]), as_bf16x8(f.b[h][pb]), acc[rb][h][pb]);
    };
    // the next half-step's LDS reads spread between this half-step's MFMAs
    constexpr int kReads = kRB + 2 * kPB, kMfma = 2 * kRB * kPB;
    constexpr int kEvery = kMfma / kReads;  // MFMAs after each read
    static_assert(kEvery >= 1, "interleave");
    auto interleave = [&]() {
#pragma unroll
      for (int i = 0; i < kReads; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, kEvery, 0);
      }
      if constexpr (kMfma > kEvery * kReads)
        __builtin_amdgcn_sched_group_barrier(0x008, kMfma - kEvery * kReads, 0);
    };

    Frag f0, f1;
    barrier_lds_drained();  // step 0 landed
    read_frag(f0, 0, 0);
    int stage = 0;
    for (int kt = 0; kt < nk; ++kt) {
      const int next = stage == STAGES - 1 ? 0 : stage + 1;
      read_frag(f1, stage, 1);
      mma(f0);
      interleave();
      __builtin_amdgcn_sched_barrier(0);
      barrier_lds_drained();  // step kt + 1 landed; this wave's reads of step kt done
      __builtin_amdgcn_sched_barrier(0);
      read_frag(f0, next, 0);
      mma(f1);
      interleave();
      __builtin_amdgcn_sched_barrier(0);
      stage = next;
    }

    // Stage the accumulators as fp32 rows in LDS: acc[rb][h][pb][i] is row
    // BM/2 wm + 16 rb + 4 g4 + i, local pair BP/2 wn + 16 pb + l16, low (h = 0) or high.
    barrier_lds_drained();  // every LDS read done, every producer load landed
    float* ep = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float* row = ep + ((BM / 2) * wm + 16 * rb + 4 * g4 + i) * kEpStride + kWP * wn + l16;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int pb = 0; pb < kPB; ++pb) row[BP * h + 16 * pb] = acc[rb][h][pb][i];
      }
    if (tid < BM) {
      int64_t* meta = reinterpret_cast<int64_t*>(smem + Sh::kEpMetaOff);
      meta[tid] = my_dq;
      meta[BM + tid] = my_dkv;
      meta[2 * BM + tid] = my_rope;
    }
    barrier_lds_drained();
  }

  // Every thread rotates and stores groups of 8 pairs of one row (16-byte stores): all the
  // LDS and sin/cos reads of its groups first, then the stores.
  const float* ep = reinterpret_cast<const float*>(smem);
  const int64_t* meta = reinterpret_cast<const int64_t*>(smem + Sh::kEpMetaOff);
  constexpr int kGroups = BP / 8, kItems = BM * kGroups;
  constexpr int kPer = (kItems + kThreads - 1) / kThreads;
  EpGroup grp[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int it = min(tid + kThreads * j, kItems - 1);
    const int row = it / kGroups, g = it - kGroups * row;
    const int p0 = BP * nt + 8 * g;
    const int mat = p0 / pairs_per_mat, rem = p0 - mat * pairs_per_mat;
    const bool mine = kItems % kThreads == 0 || tid + kThreads * j < kItems;
    grp[j].load(a, ep + row * kEpStride + 8 * g, BP, mat, rem,
                mine ? meta[(mat == 0 ? 0 : BM) + row] : -1, meta[2 * BM + row]);
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j) grp[j].store(a);
}

}  // namespace
}  // namespace fdl

namespace fdl {
namespace {

// Launch plan by row count (measured on MI355X at d_model 4096): up to 128 rows the
// projection streams the weights (32-pair tiles, 192 workgroups, 6-8 stages: 18.6 us at
// 40 rows, 23 us at 128); above that the wide tiles keep the MFMAs fed (128 x 32-pair
// tiles take 45 us at 192 rows against 36 us for the wide tiles).
struct QkvPlan {
  void (*kernel)(QkvArgs);
  int bm;       // rows per tile
  int bp;       // pairs per tile
  int threads;  // per workgroup
};

constexpr int kPcBM = 128, kPcBP = 96;

template <int BM, int BP, int NPROD, int STAGES>
constexpr QkvPlan pc_plan() {
  return {qkv_pc_kernel<BM, BP, NPROD, STAGES>, BM, BP, PcShape<BM, BP, NPROD, STAGES>::kThreads};
}

QkvPlan qkv_plan(int64_t n_rows) {
  if (n_rows <= 64) return pc_plan<64, 32, 4, 8>();
  if (n_rows <= 128) return pc_plan<128, 32, 4, 6>();
  return pc_plan<kPcBM, kPcBP, 4, 4>();
}

// Compute units of the current device (cached per device).
int device_cus() {
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

// Rows handed to the weight-streaming kernel at the end of a producer/consumer launch: a
// remainder of at most 64 rows that would otherwise open one more round of workgroups on
// the device (one workgroup per CU). At 576 rows: 4 full tiles (one round, 54 us) plus a
// 64-row stream (19 us) instead of 5 tiles in two rounds (~100 us).
int64_t qkv_tail_rows(int64_t n_rows, int64_t n_pairs) {
  if (n_rows <= kPcBM) return 0;
  const int64_t tail = n_rows % kPcBM;
  if (tail == 0 || tail > 64) return 0;
  const int64_t per_mtile = n_pairs / kPcBP;
  const int64_t cus = device_cus();
  const int64_t full = (n_rows / kPcBM) * per_mtile;
  const bool new_round = (full + per_mtile + cus - 1) / cus > (full + cus - 1) / cus;
  return new_round ? tail : 0;
}

// Launches `plan` over rows [r0, r0 + n) of the call described by `args`.
hipError_t qkv_launch(const QkvPlan& plan, QkvArgs args, int64_t r0, int64_t n,
                      hipStream_t stream) {
  const int64_t D = args.d_model;
  const int64_t n_pairs = 3 * int64_t(args.n_heads) * kHalf;  // a multiple of every plan's bp
  args.x += r0 * D;
  args.slot += r0;
  if (args.rope_row) args.rope_row += r0;
  args.q_out += r0 * D;
  if (args.kv_packed) {
    args.k_out += r0 * D;
    args.v_out += r0 * D;
    args.n_kv_rows = n;
  }
  args.n_rows = n;
  const int64_t n_mtiles = (n + plan.bm - 1) / plan.bm;
  const int64_t n_tiles = n_mtiles * (n_pairs / plan.bp);
  if (n_tiles >= (int64_t(1) << 31)) return hipErrorInvalidValue;
  args.n_mtiles = static_cast<int>(n_mtiles);
  args.n_tiles = static_cast<int>(n_tiles);
  hipLaunchKernelGGL(plan.kernel, dim3(static_cast<unsigned>(n_tiles)), dim3(plan.threads), 0,
                     stream, args);
  return hipGetLastError();
}

}  // namespace
}  // namespace fdl

extern "C" int fdl_qkv_rope_cache(const void* x, const void* wq, const void* wk,
                                  const void* wv, const float* rope_sin, const float* rope_cos,
                                  int64_t n_rope_rows, const int64_t* slot,
                                  const int64_t* rope_row, int64_t n_rows, int64_t d_model,
                                  int64_t n_heads, int64_t head_dim, void* q_out, void* k_out,
                                  void* v_out, int64_t n_kv_rows, int32_t flags,
                                  void* stream) {
  using namespace fdl;
  FDL_REQUIRE(n_rows >= 0, FDL_ERR_SHAPE, "fdl_qkv_rope_cache: n_rows = %lld < 0",
              (long long)n_rows);
  FDL_REQUIRE(head_dim == kHeadDim, FDL_ERR_UNSUPPORTED,
              "fdl_qkv_rope_cache: head_dim = %lld (only 128 is implemented)",
              (long long)head_dim);
  FDL_REQUIRE(n_heads >= 1 && d_model == n_heads * head_dim, FDL_ERR_SHAPE,
              "fdl_qkv_rope_cache: d_model (%lld) != n_heads (%lld) * head_dim",
              (long long)d_model, (long long)n_heads);
  FDL_REQUIRE(d_model <= (1 << 16), FDL_ERR_UNSUPPORTED,
              "fdl_qkv_rope_cache: d_model = %lld too large", (long long)d_model);
  FDL_REQUIRE(d_model % kDAlign == 0, FDL_ERR_UNSUPPORTED,
              "fdl_qkv_rope_cache: d_model = %lld is not a multiple of %d", (long long)d_model,
              kDAlign);
  FDL_REQUIRE((flags & ~(FDL_QKV_KV_PACKED | FDL_QKV_ROPE_HALVES_EQUAL)) == 0, FDL_ERR_SHAPE,
              "fdl_qkv_rope_cache: flags = %d has unknown bits", flags);
  const int kv_packed = (flags & FDL_QKV_KV_PACKED) ? 1 : 0;
  FDL_REQUIRE(!kv_packed || n_kv_rows == n_rows, FDL_ERR_SHAPE,
              "fdl_qkv_rope_cache: packed K/V needs n_kv_rows == n_rows");
  FDL_REQUIRE(n_kv_rows >= 0 && n_rope_rows >= 0, FDL_ERR_SHAPE,
              "fdl_qkv_rope_cache: negative table size");
  if (n_rows == 0) return ok();
  FDL_REQUIRE_PTR(x);
  FDL_REQUIRE_PTR(wq);
  FDL_REQUIRE_PTR(wk);
  FDL_REQUIRE_PTR(wv);
  FDL_REQUIRE_PTR(rope_sin);
  FDL_REQUIRE_PTR(rope_cos);
  FDL_REQUIRE_PTR(slot);
  FDL_REQUIRE_PTR(q_out);
  FDL_REQUIRE_PTR(k_out);
  FDL_REQUIRE_PTR(v_out);
  FDL_REQUIRE_ALIGNED(x, 16);
  FDL_REQUIRE_ALIGNED(wq, 16);
  FDL_REQUIRE_ALIGNED(wk, 16);
  FDL_REQUIRE_ALIGNED(wv, 16);
  FDL_REQUIRE_ALIGNED(rope_sin, 16);
  FDL_REQUIRE_ALIGNED(rope_cos, 16);
  FDL_REQUIRE_ALIGNED(q_out, 16);
  FDL_REQUIRE_ALIGNED(k_out, 16);
  FDL_REQUIRE_ALIGNED(v_out, 16);
  FDL_REQUIRE((n_rows + 63) / 64 * (3 * n_heads * kHalf / 32) < (int64_t(1) << 31),
              FDL_ERR_UNSUPPORTED, "fdl_qkv_rope_cache: %lld rows is too many",
              (long long)n_rows);
  QkvArgs args;
  args.x = static_cast<const uint16_t*>(x);
  args.w[0] = static_cast<const uint16_t*>(wq);
  args.w[1] = static_cast<const uint16_t*>(wk);
  args.w[2] = static_cast<const uint16_t*>(wv);
  args.sin = rope_sin;
  args.cos = rope_cos;
  args.slot = slot;
  args.rope_row = rope_row;
  args.q_out = static_cast<uint16_t*>(q_out);
  args.k_out = static_cast<uint16_t*>(k_out);
  args.v_out = static_cast<uint16_t*>(v_out);
  args.n_rows = n_rows;
  args.n_rope_rows = n_rope_rows;
  args.n_kv_rows = n_kv_rows;
  args.d_model = static_cast<int>(d_model);
  args.n_heads = static_cast<int>(n_heads);
  args.n_mtiles = 0;
  args.n_tiles = 0;
  args.kv_packed = kv_packed;
  args.rope_half = (flags & FDL_QKV_ROPE_HALVES_EQUAL) ? 1 : 0;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t tail = qkv_tail_rows(n_rows, 3 * n_heads * kHalf);
  const int64_t head = n_rows - tail;
  FDL_HIP_CHECK(qkv_launch(qkv_plan(head), args, 0, head, st));
  if (tail > 0) FDL_HIP_CHECK(qkv_launch(qkv_plan(tail), args, head, tail, st));
  return ok();
}
