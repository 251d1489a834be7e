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
// Two kernels, chosen by the number of rows:
//  * qkv_pc_kernel (more than 64 rows): 128 rows x 96 pairs per workgroup (512 rows: one
//    tile per CU). Sixteen wavefronts in two roles: four producers move the X and W tiles
//    of each 64-wide reduction step straight from global memory into LDS (global_load_lds,
//    three LDS stages in flight), and twelve consumers (three per SIMD) run the 16x16x32
//    MFMAs from LDS. A consumer never issues a global memory instruction, so it is never
//    held behind the texture-address queue, and the three consumers of a SIMD hide each
//    other's LDS latency.
//  * qkv_stream_kernel<BM, BP> (up to 64 rows, weight streaming): 64 rows x 32 pairs per
//    workgroup so the launch covers the CUs; X and W tiles staged through LDS with the
//    global loads kStages steps ahead in a ring of registers and the LDS fragment reads of
//    the next half-step interleaved with the MFMAs of the current one.
#include <atomic>
#include <type_traits>

#include "fdl_device.h"
#include "fdl_host.h"

namespace fdl {
namespace {

constexpr int kHeadDim = 128;
constexpr int kHalf = 64;
constexpr int kKT = 64;  // reduction step, bf16 elements (8 chunks of 16 B per row)
constexpr int kThreads = 256;
constexpr int kStages = 4;  // reduction steps in flight (register ring); even

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
};

// Chunk c (16 B) of LDS row r is stored at chunk c ^ ((r >> 1) & 7) of that row: two
// 128-byte rows share one 256-byte bank line, so 16 consecutive rows read at the same
// logical chunk land on 16 distinct 4-bank groups.
__device__ __forceinline__ int swz(int r, int c) { return r * 8 + (c ^ ((r >> 1) & 7)); }

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

// Destination rows of tile rows m0 .. m0 + BM - 1, written by threads 0 .. BM - 1:
// dst[0] = Q row, dst[1] = K/V row (cache slot, or the packed row), rope = sin/cos row.
// A row past n_rows, or with an out-of-range slot or rope row, gets -1 (skipped in all
// three outputs).
template <int BM>
__device__ __forceinline__ void tile_rows(const QkvArgs& a, int64_t m0, int64_t (&dst)[2][BM],
                                          int64_t (&rope)[BM]) {
  const int tid = threadIdx.x;
  if (tid < BM) {
    const int64_t r = m0 + tid;
    int64_t dq = -1, dkv = -1, rr_ok = -1;
    if (r < a.n_rows) {
      const int64_t s = a.slot[r];
      const int64_t rr = a.rope_row ? a.rope_row[r] : s;
      const bool rope_ok = rr >= 0 && rr < a.n_rope_rows;
      const bool slot_ok = a.kv_packed || (s >= 0 && s < a.n_kv_rows);
      if (rope_ok && slot_ok) {
        dq = r;
        dkv = a.kv_packed ? r : s;
        rr_ok = rr;
      }
    }
    dst[0][tid] = dq;
    dst[1][tid] = dkv;
    rope[tid] = rr_ok;
  }
}

// Rotates (lo, hi) = (q~_c, q~_{c+64}) of one row and stores the bf16 pair.
__device__ __forceinline__ void store_pair(const QkvArgs& a, int mat, int64_t dst, int64_t rope,
                                           int head, int c, float lo, float hi) {
  if (mat < 2) {
    const float* sn = a.sin + rope * kHeadDim;
    const float* cs = a.cos + rope * kHeadDim;
    const float s1 = sn[c], s2 = sn[c + kHalf], c1 = cs[c], c2 = cs[c + kHalf];
    const float rlo = lo * c1 - hi * s1;
    const float rhi = hi * c2 + lo * s2;
    lo = rlo;
    hi = rhi;
  }
  uint16_t* base = mat == 0 ? a.q_out : (mat == 1 ? a.k_out : a.v_out);
  uint16_t* d = base + dst * a.d_model + int64_t(head) * kHeadDim;
  d[c] = f2bf(lo);
  d[c + kHalf] = f2bf(hi);
}

// ---------------------------------------------------------------------------------------
// qkv_stream_kernel: BM rows x BP pairs per workgroup; wavefront (wm, wn) owns rows
// BM/2 * wm .. + BM/2 and pairs BP/2 * wn .. + BP/2 (low and high columns).
template <int BM, int BP, int OCC>
__global__ __launch_bounds__(kThreads, OCC) void qkv_stream_kernel(QkvArgs a) {
  constexpr int kWP = BP / 2;               // pairs per wavefront
  constexpr int kPB = kWP / 16;             // 16-pair MFMA blocks per wavefront
  constexpr int kRB = BM / 32;              // 16-row MFMA blocks per wavefront
  constexpr int kXLd = BM * 8 / kThreads;   // X chunks per thread per step
  constexpr int kWLd = 2 * BP * 8 / kThreads;  // W chunks per thread per step
  static_assert(kPB >= 1 && kRB >= 1 && kXLd >= 1 && kWLd >= 1, "tile too small");
  __shared__ u32x4 As[2][BM * 8];
  __shared__ u32x4 Bs[2][2 * BP * 8];  // rows 0 .. BP-1: low columns; BP .. 2BP-1: high
  __shared__ int64_t s_dst[2][BM];
  __shared__ int64_t s_rope[BM];

  const int tid = threadIdx.x;
  int nt, mt;
  tile_coords(xcd_tile(blockIdx.x, a.n_tiles), a.n_mtiles, a.n_tiles, nt, mt);
  const int64_t m0 = int64_t(mt) * BM;
  const int D = a.d_model;
  const int pairs_per_mat = a.n_heads * kHalf;
  tile_rows<BM>(a, m0, s_dst, s_rope);

  // Global -> LDS staging sources. Tile rows past n_rows load row n_rows - 1 (never
  // stored), so every load is unconditional and the compiler's wait counts stay exact.
  const uint16_t* xsrc[kXLd];
  const uint16_t* wsrc[kWLd];
  int xdst[kXLd], wdst[kWLd];
#pragma unroll
  for (int i = 0; i < kXLd; ++i) {
    const int id = tid + kThreads * i, row = id >> 3, c = id & 7;
    const int64_t r = min(m0 + row, a.n_rows - 1);
    xsrc[i] = a.x + r * D + 8 * c;
    xdst[i] = swz(row, c);
  }
#pragma unroll
  for (int i = 0; i < kWLd; ++i) {
    const int id = tid + kThreads * i, row = id >> 3, c = id & 7;
    const int hlf = row / BP, p = BP * nt + (row - hlf * BP);
    const int mat = p / pairs_per_mat, rem = p - mat * pairs_per_mat;
    wsrc[i] = a.w[mat] + int64_t((rem >> 6) * kHeadDim + (rem & 63) + kHalf * hlf) * D + 8 * c;
    wdst[i] = swz(row, c);
  }
  struct Stage {
    u32x4 x[kXLd], w[kWLd];
  };
  Stage ring[kStages];
  const int nk = D / kKT;  // a multiple of kStages (checked on the host)
  // Steps past the end re-read the last step (never committed).
  auto issue = [&](Stage& st, int kt) {
    const int k0 = min(kt, nk - 1) * kKT;
#pragma unroll
    for (int i = 0; i < kXLd; ++i) st.x[i] = ld16(xsrc[i] + k0);
#pragma unroll
    for (int i = 0; i < kWLd; ++i) st.w[i] = ld16(wsrc[i] + k0);
  };
  auto commit = [&](const Stage& st, int buf) {
#pragma unroll
    for (int i = 0; i < kXLd; ++i) As[buf][xdst[i]] = st.x[i];
#pragma unroll
    for (int i = 0; i < kWLd; ++i) Bs[buf][wdst[i]] = st.w[i];
  };

  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int l16 = lane & 15, g4 = lane >> 4;
  // MFMA operands of one 32-wide half-step ss of a step: lane (l16, g4) takes chunk
  // 4 * ss + g4 of its row.
  struct Frag {
    bf16x8 a[kRB];
    bf16x8 b[2][kPB];
  };
  auto read_frag = [&](Frag& f, int buf, int ss) {
    const int c = 4 * ss + g4;
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb)
      f.a[rb] = as_bf16x8(As[buf][swz((BM / 2) * wm + 16 * rb + l16, c)]);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int pb = 0; pb < kPB; ++pb)
        f.b[h][pb] = as_bf16x8(Bs[buf][swz(BP * h + kWP * wn + 16 * pb + l16, c)]);
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
          acc[rb][h][pb] = mfma16(f.a[rb], f.b[h][pb], acc[rb][h][pb]);
  };
  // Instruction groups for one half-step: the LDS fragment reads and the LDS writes (first
  // half) or global loads (second half) are spread between the MFMAs.
  constexpr int kMfma = 2 * kRB * kPB;
  constexpr int kMem = kXLd + kWLd;
  auto interleave = [&](auto mem_mask) {
    if constexpr (kMfma >= 2 * kMem) {
#pragma unroll
      for (int i = 0; i < kMem; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(decltype(mem_mask)::value, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, kMfma - 2 * kMem, 0);
    }
  };

  Frag f0, f1;
#pragma unroll
  for (int s = 0; s < kStages; ++s) {
    issue(ring[s], s);
    __builtin_amdgcn_sched_barrier(0);
  }
  commit(ring[0], 0);
  __syncthreads();
  read_frag(f0, 0, 0);
  __builtin_amdgcn_sched_barrier(0);
  issue(ring[0], kStages);
  __builtin_amdgcn_sched_barrier(0);
  // Step kt: f0 holds half-step 0 (read earlier), LDS buffer kt & 1 holds the step, ring
  // slot (kt + 1) % kStages holds step kt + 1 in registers.
  for (int kt0 = 0; kt0 < nk; kt0 += kStages) {
#pragma unroll
    for (int j = 0; j < kStages; ++j) {
      const int kt = kt0 + j;
      const int buf = j & 1;  // kStages is even
      // half-step 0: read half-step 1, store step kt + 1 to the other buffer (its last
      // reads were before the previous barrier), MFMAs of half-step 0
      read_frag(f1, buf, 1);
      commit(ring[(j + 1) % kStages], buf ^ 1);
      mma(f0);
      interleave(std::integral_constant<int, 0x200>{});  // LDS write
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
      // half-step 1: read half-step 0 of step kt + 1, refill the ring slot, MFMAs
      read_frag(f0, buf ^ 1, 0);
      issue(ring[(j + 1) % kStages], kt + 1 + kStages);
      mma(f1);
      interleave(std::integral_constant<int, 0x020>{});  // global load
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Epilogue: acc[rb][h][pb][i] is row BM/2 * wm + 16 rb + 4 g4 + i, pair
  // BP * nt + kWP * wn + 16 pb + l16, low (h = 0) or high (h = 1) column.
#pragma unroll
  for (int pb = 0; pb < kPB; ++pb) {
    const int p = BP * nt + kWP * wn + 16 * pb + l16;
    const int mat = p / pairs_per_mat, rem = p - mat * pairs_per_mat;
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = (BM / 2) * wm + 16 * rb + 4 * g4 + i;
        const int64_t dst = s_dst[mat == 0 ? 0 : 1][row];
        if (dst < 0) continue;
        store_pair(a, mat, dst, s_rope[row], rem >> 6, rem & 63, acc[rb][0][pb][i],
                   acc[rb][1][pb][i]);
      }
  }
}

// ---------------------------------------------------------------------------------------
// qkv_pc_kernel: 128 rows x 96 pairs; consumer wavefront (wm, wn), wm < 4, wn < 3, owns rows
// 32 wm .. + 32 and pairs 32 wn .. + 32 (low and high columns).
constexpr int kPcBM = 128;
constexpr int kPcBP = 96;
constexpr int kPcThreads = 1024;  // 12 consumer + 4 producer wavefronts
constexpr int kPcStages = 3;                         // LDS stages
constexpr int kPcABytes = kPcBM * 128;               // X tile of one step (16 KB)
constexpr int kPcStageBytes = kPcABytes + 2 * kPcBP * 128;  // + W tile (24 KB)
constexpr int kPcLoads = kPcStageBytes / 1024 / 4;   // 1 KB loads per producer per step

typedef __attribute__((address_space(3))) void* lds_ptr;
typedef __attribute__((address_space(1))) void* glb_ptr;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Workgroup barrier without the compiler's memory fence; each side waits for exactly the
// memory operations it must (the fence would drain every outstanding global load).
__device__ __forceinline__ void barrier_lds_drained() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
__device__ __forceinline__ void barrier_only() { asm volatile("s_barrier" ::: "memory"); }

__global__ __launch_bounds__(kPcThreads, 1) void qkv_pc_kernel(QkvArgs a) {
  constexpr int kWP = kPcBP / 3, kPB = kWP / 16;
  __shared__ __align__(1024) uint8_t smem[kPcStages * kPcStageBytes];
  __shared__ int64_t s_dst[2][kPcBM];
  __shared__ int64_t s_rope[kPcBM];

  const int tid = threadIdx.x;
  int nt, mt;
  tile_coords(xcd_tile(blockIdx.x, a.n_tiles), a.n_mtiles, a.n_tiles, nt, mt);
  const int64_t m0 = int64_t(mt) * kPcBM;
  const int D = a.d_model;
  const int pairs_per_mat = a.n_heads * kHalf;
  tile_rows<kPcBM>(a, m0, s_dst, s_rope);
  // The wavefront index is uniform; readfirstlane makes the role test a scalar branch, so a
  // wavefront executes only its own role's barriers (both roles execute 1 + nk of them).
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const bool producer = wave >= 12;
  const int pw = wave - 12;
  const int nk = D / kKT;

  if (producer) {
    // Load i of producer pw fills LDS bytes [1024 q, 1024 q + 1024) of the step's tile
    // (q = 8-row block): lane -> row 8 q + lane / 8, LDS chunk lane % 8, which holds the
    // row's logical chunk (lane % 8) ^ ((row >> 1) & 7) (the swz() layout). Tile rows past
    // n_rows re-read row n_rows - 1 (never stored).
    const uint16_t* src[kPcLoads];
    int dst_off[kPcLoads];
#pragma unroll
    for (int i = 0; i < kPcLoads; ++i) {
      const int q = kPcLoads * pw + i;
      const int row = 8 * q + (lane >> 3);
      const int c = (lane & 7) ^ ((row >> 1) & 7);
      if (row < kPcBM) {
        src[i] = a.x + min(m0 + row, a.n_rows - 1) * D + 8 * c;
      } else {
        const int wr = row - kPcBM, hlf = wr / kPcBP;
        const int p = kPcBP * nt + (wr - hlf * kPcBP);
        const int mat = p / pairs_per_mat, rem = p - mat * pairs_per_mat;
        src[i] = a.w[mat] + int64_t((rem >> 6) * kHeadDim + (rem & 63) + kHalf * hlf) * D +
                 8 * c;
      }
      dst_off[i] = 1024 * q;
    }
    // Steps past the end re-read the last step into a stage nobody reads any more.
    auto issue = [&](int kt, int stage) {
      const int k0 = min(kt, nk - 1) * kKT;
      uint8_t* st = smem + stage * kPcStageBytes;
#pragma unroll
      for (int i = 0; i < kPcLoads; ++i)
        __builtin_amdgcn_global_load_lds((glb_ptr)(src[i] + k0), (lds_ptr)(st + dst_off[i]), 16,
                                         0, 0);
    };
    issue(0, 0);
    issue(1, 1);
    issue(2, 2);
    wait_vmcnt<2 * kPcLoads>();  // step 0 landed
    barrier_only();
    int stage = 0;
    for (int kt = 0; kt < nk; ++kt) {
      wait_vmcnt<kPcLoads>();  // step kt + 1 landed (step kt + 2 may still be in flight)
      barrier_only();
      issue(kt + kPcStages, stage);  // this stage's last reads came before the barrier
      stage = stage == kPcStages - 1 ? 0 : stage + 1;
    }
    wait_vmcnt<0>();  // no load may still be writing LDS when the workgroup ends
    return;
  }

  const int wm = wave / 3, wn = wave - 3 * (wave / 3);  // rows 32 wm .., pairs 32 wn ..
  const int l16 = lane & 15, g4 = lane >> 4;
  const int sw = (l16 >> 1) & 7;
  struct Frag {
    u32x4 a[2];
    u32x4 b[2][kPB];
  };
  // MFMA operands of half-step ss of the step in `stage`: lane (l16, g4) takes logical chunk
  // 4 ss + g4 of its row.
  auto read_frag = [&](Frag& f, int stage, int ss) {
    const u32x4* st = reinterpret_cast<const u32x4*>(smem + stage * kPcStageBytes);
    const int c = (4 * ss + g4) ^ sw;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) f.a[rb] = st[(32 * wm + 16 * rb + l16) * 8 + c];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int pb = 0; pb < kPB; ++pb)
        f.b[h][pb] = st[kPcABytes / 16 + (kPcBP * h + kWP * wn + 16 * pb + l16) * 8 + c];
  };
  f32x4 acc[2][2][kPB];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int pb = 0; pb < kPB; ++pb) acc[rb][h][pb] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto mma = [&](const Frag& f) {
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int pb = 0; pb < kPB; ++pb)
          acc[rb][h][pb] = mfma16(as_bf16x8(f.a[rb]), as_bf16x8(f.b[h][pb]), acc[rb][h][pb]);
  };
  // one LDS read between two MFMAs
  auto interleave = [&]() {
#pragma unroll
    for (int i = 0; i < 2 + 2 * kPB; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4 * kPB - (2 + 2 * kPB), 0);
  };

  Frag f0, f1;
  barrier_lds_drained();  // row metadata stored; step 0 landed
  read_frag(f0, 0, 0);
  int stage = 0;
  for (int kt = 0; kt < nk; ++kt) {
    const int next = stage == kPcStages - 1 ? 0 : stage + 1;
    read_frag(f1, stage, 1);
    mma(f0);
    interleave();
    __builtin_amdgcn_sched_barrier(0);
    barrier_lds_drained();  // step kt + 1 landed; this wave's reads of step kt - 2 done
    __builtin_amdgcn_sched_barrier(0);
    read_frag(f0, next, 0);
    mma(f1);
    interleave();
    __builtin_amdgcn_sched_barrier(0);
    stage = next;
  }

  // Epilogue: acc[rb][h][pb][i] is row 32 wm + 16 rb + 4 g4 + i, pair
  // 96 nt + 32 wn + 16 pb + l16, low (h = 0) or high (h = 1) column.
#pragma unroll
  for (int pb = 0; pb < kPB; ++pb) {
    const int p = kPcBP * nt + kWP * wn + 16 * pb + l16;
    const int mat = p / pairs_per_mat, rem = p - mat * pairs_per_mat;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 32 * wm + 16 * rb + 4 * g4 + i;
        const int64_t dst = s_dst[mat == 0 ? 0 : 1][row];
        if (dst < 0) continue;
        store_pair(a, mat, dst, s_rope[row], rem >> 6, rem & 63, acc[rb][0][pb][i],
                   acc[rb][1][pb][i]);
      }
  }
}

}  // namespace
}  // namespace fdl

namespace fdl {
namespace {

// Launch plan by row count (measured on MI355X at d_model 4096): up to 64 rows the
// projection streams the weights (the narrow tiles give every CU work); above that the
// producer/consumer kernel's wide tiles keep the MFMAs fed.
struct QkvPlan {
  void (*kernel)(QkvArgs);
  int bm;       // rows per tile
  int bp;       // pairs per tile
  int threads;  // per workgroup
};

QkvPlan qkv_plan(int64_t n_rows) {
  if (n_rows <= 64) return {qkv_stream_kernel<64, 32, 2>, 64, 32, kThreads};
  return {qkv_pc_kernel, kPcBM, kPcBP, kPcThreads};
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
// 64-row stream (22 us) instead of 5 tiles in two rounds (108 us).
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
                                  void* v_out, int64_t n_kv_rows, int32_t kv_packed,
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
  FDL_REQUIRE(d_model % (kKT * kStages) == 0, FDL_ERR_UNSUPPORTED,
              "fdl_qkv_rope_cache: d_model = %lld is not a multiple of %d", (long long)d_model,
              kKT * kStages);
  FDL_REQUIRE(kv_packed == 0 || kv_packed == 1, FDL_ERR_SHAPE,
              "fdl_qkv_rope_cache: kv_packed must be 0 or 1");
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
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t tail = qkv_tail_rows(n_rows, 3 * n_heads * kHalf);
  const int64_t head = n_rows - tail;
  FDL_HIP_CHECK(qkv_launch(qkv_plan(head), args, 0, head, st));
  if (tail > 0) FDL_HIP_CHECK(qkv_launch(qkv_plan(tail), args, head, tail, st));
  return ok();
}
