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
// Tiling. One workgroup (4 wavefronts) computes a 128-row x 128-column tile whose columns
// are one head of one of the three matrices, i.e. all 64 RoPE pairs (c, c + 64) of that
// head. Wavefront (wm, wn) owns rows 64*wm .. 64*wm+63 and pair columns 32*wn .. 32*wn+31;
// it runs 32x32x16 MFMAs on the low block (columns 32*wn + j) and on the high block
// (columns 64 + 32*wn + j), so lane l holds both members of pair 32*wn + (l % 32) for
// the same rows and RoPE is applied in registers before the bf16 stores. The reduction
// runs in 64-wide steps staged through LDS (double-buffered, XOR-swizzled 16-byte chunks);
// the global loads run kStages steps ahead of the MFMAs in a ring of register sets.
#include "fdl_device.h"
#include "fdl_host.h"

namespace fdl {
namespace {

constexpr int kHeadDim = 128;
constexpr int kHalf = 64;
constexpr int kBM = 128;  // rows per tile
constexpr int kBN = 128;  // output columns per tile (one head of one matrix)
constexpr int kKT = 64;   // reduction step, bf16 elements (8 chunks of 16 B per row)
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

// Two workgroups per CU (registers capped at 256 per lane).
__global__ __launch_bounds__(kThreads, 2) void qkv_rope_kernel(QkvArgs a) {
  __shared__ u32x4 As[2][kBM * 8];
  __shared__ u32x4 Bs[2][kBN * 8];
  __shared__ int64_t s_dst[kBM];   // K/V destination row per tile row (-1: skip)
  __shared__ int64_t s_rope[kBM];  // sin/cos row per tile row (-1: skip)

  const int tid = threadIdx.x;
  // Workgroup i runs on XCD i % 8. Renumber so that each XCD gets a contiguous run of
  // tiles: the m-tiles that share one weight slice then run on one XCD and share its L2.
  int t = blockIdx.x;
  if ((a.n_tiles & 7) == 0) t = (t & 7) * (a.n_tiles >> 3) + (t >> 3);
  const int ns = t / a.n_mtiles;  // n-slice = matrix * n_heads + head
  const int mt = t - ns * a.n_mtiles;
  const int mat = ns / a.n_heads;
  const int h = ns - mat * a.n_heads;
  const int64_t m0 = int64_t(mt) * kBM;
  const int D = a.d_model;
  const uint16_t* __restrict__ W = a.w[mat] + int64_t(h) * kHeadDim * D;

  if (tid < kBM) {
    const int64_t r = m0 + tid;
    int64_t dst = -1, rope = -1;
    if (r < a.n_rows) {
      // A row with an out-of-range slot or rope row is skipped in all three outputs.
      const int64_t s = a.slot[r];
      const int64_t rr = a.rope_row ? a.rope_row[r] : s;
      const bool rope_ok = rr >= 0 && rr < a.n_rope_rows;
      const bool slot_ok = a.kv_packed || (s >= 0 && s < a.n_kv_rows);
      if (rope_ok && slot_ok) {
        dst = (mat == 0 || a.kv_packed) ? r : s;  // Q is always packed by row
        rope = rr;
      }
    }
    s_dst[tid] = dst;
    s_rope[tid] = rope;
  }

  // Global -> LDS staging: each thread moves 4 chunks of the X tile and 4 of the W tile
  // per 64-wide step. kStages steps are in flight in a ring of register sets, so a step's
  // loads have kStages steps of MFMA work to land before they are written to LDS. Tile
  // rows past n_rows load row n_rows - 1 instead (their results are never stored): the
  // loads stay unconditional, which keeps the compiler's memory wait counts exact.
  int ld_row[4], ld_c[4];
  const uint16_t* xrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int id = tid + kThreads * i;
    ld_row[i] = id >> 3;
    ld_c[i] = id & 7;
    const int64_t r = min(m0 + ld_row[i], a.n_rows - 1);
    xrow[i] = a.x + r * D + 8 * ld_c[i];
  }
  struct Stage {
    u32x4 a[4], b[4];
  };
  Stage rs[kStages];
  auto issue = [&](Stage& st, int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      st.a[i] = ld16(xrow[i] + k0);
      st.b[i] = ld16(W + int64_t(ld_row[i]) * D + k0 + 8 * ld_c[i]);
    }
  };
  auto commit = [&](const Stage& st, int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      As[buf][swz(ld_row[i], ld_c[i])] = st.a[i];
      Bs[buf][swz(ld_row[i], ld_c[i])] = st.b[i];
    }
  };

  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, g = lane >> 5;
  const int arow0 = 64 * wm + l32, arow1 = arow0 + 32;
  const int bcol0 = 32 * wn + l32, bcol1 = bcol0 + kHalf;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  auto compute = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < kKT / 16; ++ks) {
      const int c = 2 * ks + g;  // this lane's 8 reduction elements of the 16-wide step
      const bf16x8 a0 = as_bf16x8(As[buf][swz(arow0, c)]);
      const bf16x8 a1 = as_bf16x8(As[buf][swz(arow1, c)]);
      const bf16x8 b0 = as_bf16x8(Bs[buf][swz(bcol0, c)]);
      const bf16x8 b1 = as_bf16x8(Bs[buf][swz(bcol1, c)]);
      acc[0][0] = mfma32(a0, b0, acc[0][0]);
      acc[0][1] = mfma32(a0, b1, acc[0][1]);
      acc[1][0] = mfma32(a1, b0, acc[1][0]);
      acc[1][1] = mfma32(a1, b1, acc[1][1]);
    }
  };

  // Step t is loaded into rs[t % kStages] and written to LDS buffer t & 1 after step t - 1
  // is computed. Steps past the end re-read the last step (an L2 hit) and are never
  // committed.
  const int nk = D / kKT;  // a multiple of kStages (checked on the host)
  auto step_k0 = [&](int t) { return min(t, nk - 1) * kKT; };
#pragma unroll
  for (int st = 0; st < kStages; ++st) issue(rs[st], step_k0(st));
  commit(rs[0], 0);
  __syncthreads();
  issue(rs[0], step_k0(kStages));
  for (int kt0 = 0; kt0 < nk; kt0 += kStages) {
#pragma unroll
    for (int j = 0; j < kStages; ++j) {
      const int kt = kt0 + j;  // LDS buffer kt & 1 == j & 1 since kStages is even
      compute(j & 1);
      if (kt + 1 < nk) commit(rs[(j + 1) % kStages], (j + 1) & 1);
      __syncthreads();
      issue(rs[(j + 1) % kStages], step_k0(kt + 1 + kStages));
    }
  }

  // Epilogue: RoPE in registers, bf16 stores straight to Q / the cache rows.
  uint16_t* __restrict__ dst_base = mat == 0 ? a.q_out : (mat == 1 ? a.k_out : a.v_out);
  const int p = 32 * wn + l32;  // pair index within the head
#pragma unroll
  for (int rb2 = 0; rb2 < 2; ++rb2) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = 64 * wm + 32 * rb2 + 8 * (e >> 2) + 4 * g + (e & 3);
      const int64_t dst = s_dst[row];
      if (dst < 0) continue;
      float lo = acc[rb2][0][e], hi = acc[rb2][1][e];
      if (mat < 2) {
        const float* sn = a.sin + s_rope[row] * kHeadDim;
        const float* cs = a.cos + s_rope[row] * kHeadDim;
        const float s1 = sn[p], s2 = sn[p + kHalf], c1 = cs[p], c2 = cs[p + kHalf];
        const float rlo = lo * c1 - hi * s1;
        const float rhi = hi * c2 + lo * s2;
        lo = rlo;
        hi = rhi;
      }
      uint16_t* d = dst_base + dst * D + int64_t(h) * kHeadDim;
      d[p] = f2bf(lo);
      d[p + kHalf] = f2bf(hi);
    }
  }
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
  const int64_t n_mtiles = (n_rows + kBM - 1) / kBM;
  const int64_t n_tiles = n_mtiles * 3 * n_heads;
  FDL_REQUIRE(n_tiles < (int64_t(1) << 31), FDL_ERR_UNSUPPORTED,
              "fdl_qkv_rope_cache: %lld rows is too many", (long long)n_rows);
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
  args.n_mtiles = static_cast<int>(n_mtiles);
  args.n_tiles = static_cast<int>(n_tiles);
  args.kv_packed = kv_packed;
  hipLaunchKernelGGL(qkv_rope_kernel, dim3(static_cast<unsigned>(n_tiles)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), args);
  FDL_HIP_CHECK(hipGetLastError());
  return ok();
}
