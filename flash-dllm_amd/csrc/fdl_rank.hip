// Importance ranking of decoded slots and top-k gather of the tracked refresh set.
//
// Follows generate.py:364-366 (`full_pos[j, :nd-keep]` re-ordered by an ascending sort of
// attn_scores) and generate.py:375-381 (the tracked set is the tail of that order, i.e.
// the highest-scoring slots). The reference's torch.sort is unstable; here ties are
// resolved so that among equal scores the lower slot ranks higher (it sits later in the
// ascending order), which makes the result a total order.
//
// One workgroup per segment. Each entry becomes a 64-bit key
//   (orderable(score) << 32) | (0xffffffff - slot)
// whose ascending order is (score ascending, slot descending); the segment is padded to
// T * R keys (T threads, R keys each, a power of two) with all-ones keys (they sort last) and
// bitonic-sorted with thread t holding keys t*R .. t*R + R - 1 in registers. The network is
// unrolled at compile time: compare-exchange steps whose stride is below R run inside a
// thread, strides R .. 32R are lane exchanges within a wavefront (DPP quad permutes for
// lanes 1 and 2 apart, ds_swizzle for 4, 8 and 16, a lane permute for 32), and only the
// strides of 64R and above go through LDS with a workgroup barrier (10 of the 55 steps for
// 1024 keys with 1024 threads of one key).
//
// rank_kernel<T, R, true> (fdl_importance_accumulate_rank) first does, for the sequence
// of its segment, what fdl_importance_accumulate does for that sequence's keys (page-table
// order, so the per-head loads are coalesced; heads summed in ascending order, then one fma
// into the score), then, after a workgroup barrier, ranks the segment by the new scores:
// the step's last head reduction and its ranking in one launch.
#include "fdl_device.h"
#include "fdl_host.h"

namespace fdl {
namespace {

constexpr int kMaxLen = 8192;  // 1024 threads x 8 keys

// Monotone map float -> uint32 (x < y  <=>  ord(x) < ord(y)); -0.0 and +0.0 map together.
__device__ __forceinline__ uint32_t orderable(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) == 0) u = 0;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// The value of lane (lane ^ M) of the wavefront.
template <int M>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
  const int x = static_cast<int>(v);
  if constexpr (M == 1) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
  } else if constexpr (M == 2) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
  } else if constexpr (M == 4 || M == 8 || M == 16) {
    // bit mode: lane i of each 32-lane half reads lane ((i & 0x1f) | 0) ^ M
    return static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(x, 0x1f | (M << 10)));
  } else {
    static_assert(M == 32, "lane distance");
    return static_cast<uint32_t>(__shfl_xor(x, 32));
  }
}

template <int M>
__device__ __forceinline__ uint64_t xor_lane64(uint64_t v) {
  const uint32_t lo = xor_lane<M>(static_cast<uint32_t>(v));
  const uint32_t hi = xor_lane<M>(static_cast<uint32_t>(v >> 32));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// Keeps min or max of (mine, other) for element i of a compare-exchange at stride j within
// bitonic blocks of size k: the lower element of an ascending pair keeps the minimum.
// One 64-bit comparison and one select: mine is kept when it is the one wanted.
__device__ __forceinline__ uint64_t cx(uint64_t mine, uint64_t other, int i, int j, int k) {
  const bool lower = (i & j) == 0;
  const bool asc = (i & k) == 0;
  const bool take_min = lower == asc;
  return (mine < other) == take_min ? mine : other;
}

// One compare-exchange step (bitonic block size K, stride J) over the R keys of each thread.
template <int T, int R, int K, int J>
__device__ __forceinline__ void bitonic_step(uint64_t (&key)[R], int tid, uint64_t (*xbuf)[T * R],
                                             int& buf) {
  if constexpr (J >= 64 * R) {
    // partner in another wavefront: exchange through LDS (two buffers, so one barrier
    // separates a step's reads from the next step's writes)
#pragma unroll
    for (int r = 0; r < R; ++r) xbuf[buf][tid * R + r] = key[r];
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = tid * R + r;
      key[r] = cx(key[r], xbuf[buf][i ^ J], i, J, K);
    }
    buf ^= 1;
  } else if constexpr (J >= R) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = tid * R + r;
      key[r] = cx(key[r], xor_lane64<J / R>(key[r]), i, J, K);
    }
  } else {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int rp = r ^ J;
      if (rp > r) {
        const int i = tid * R + r;
        const uint64_t lo = cx(key[r], key[rp], i, J, K);
        const uint64_t hi = cx(key[rp], key[r], i ^ J, J, K);
        key[r] = lo;
        key[rp] = hi;
      }
    }
  }
}

template <int T, int R, int K, int J>
__device__ __forceinline__ void bitonic_merge(uint64_t (&key)[R], int tid,
                                              uint64_t (*xbuf)[T * R], int& buf) {
  bitonic_step<T, R, K, J>(key, tid, xbuf, buf);
  if constexpr (J > 1) bitonic_merge<T, R, K, J / 2>(key, tid, xbuf, buf);
}

template <int T, int R, int K>
__device__ __forceinline__ void bitonic_sort(uint64_t (&key)[R], int tid, uint64_t (*xbuf)[T * R],
                                             int& buf) {
  bitonic_merge<T, R, K, K / 2>(key, tid, xbuf, buf);
  if constexpr (K < T * R) bitonic_sort<T, R, 2 * K>(key, tid, xbuf, buf);
}

struct RankArgs {
  float* scores;  // read; written only by the accumulating variant
  int64_t n_scores;
  int64_t* slots;
  int64_t n_slot_entries;
  const int32_t* seg;
  int max_len;
  int64_t* topk_out;
  int k;
  // accumulating variant only
  const float* part;  // [n_heads][n_scores]
  int n_heads;
  float scale;
  const int32_t* page_table;  // [n_seq][max_pages]
  int n_seq;
  int max_pages;
  int page_log2;
  const int32_t* seg_keys;  // [n_seg][2]: page-table row, key count of the segment's sequence
};

// The head sum of fdl_importance_accumulate for one slot: ascending head order, loads
// issued 16 at a time (32 at once for 32 heads).
__device__ __forceinline__ float head_sum(const float* __restrict__ part, int n_heads,
                                          int64_t n_scores, int64_t slot) {
  float sum = 0.f;
  int h = 0;
  if (n_heads == 32) {
    float v[32];
#pragma unroll
    for (int u = 0; u < 32; ++u) v[u] = part[int64_t(u) * n_scores + slot];
#pragma unroll
    for (int u = 0; u < 32; ++u) sum += v[u];
    return sum;
  }
  for (; h + 16 <= n_heads; h += 16) {
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = part[int64_t(h + u) * n_scores + slot];
#pragma unroll
    for (int u = 0; u < 16; ++u) sum += v[u];
  }
  for (; h < n_heads; ++h) sum += part[int64_t(h) * n_scores + slot];
  return sum;
}

template <int T, int R, bool kAcc>
__global__ __launch_bounds__(T) void rank_kernel(RankArgs a) {
  constexpr int P = T * R;
  float* __restrict__ scores = a.scores;
  const int64_t n_scores = a.n_scores;
  int64_t* slots = a.slots;
  const int64_t n_slot_entries = a.n_slot_entries;
  const int32_t* __restrict__ seg = a.seg;
  const int max_len = a.max_len;
  int64_t* topk_out = a.topk_out;
  const int k = a.k;
  const int tid = threadIdx.x;

  __shared__ uint64_t xbuf[2][P];
  const int s = blockIdx.x;
  const int64_t start = seg[2 * s];
  int len = seg[2 * s + 1];
  // a segment longer than max_len (rejected by the host) is left as is
  if (start < 0 || len < 0 || len > max_len || len > P || start + len > n_slot_entries) len = 0;
  // the segment's slots (their loads overlap the reduction below)
  int64_t slot_r[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = tid * R + r;
    slot_r[r] = i < len ? slots[start + i] : -1;
  }

  if constexpr (kAcc) {
    const int b = a.seg_keys[2 * blockIdx.x], k_end = a.seg_keys[2 * blockIdx.x + 1];
    // a row or key count out of range (rejected by the host) accumulates nothing
    if (b >= 0 && b < a.n_seq && k_end > 0 &&
        int64_t(k_end) <= (int64_t(a.max_pages) << a.page_log2)) {
      const int32_t* ptab = a.page_table + int64_t(b) * a.max_pages;
      const int pmask = (1 << a.page_log2) - 1;
      for (int n = tid; n < k_end; n += T) {
        const int64_t sl = (int64_t(ptab[n >> a.page_log2]) << a.page_log2) | (n & pmask);
        if (sl < 0 || sl >= n_scores) continue;
        scores[sl] = __builtin_fmaf(a.scale, head_sum(a.part, a.n_heads, n_scores, sl), scores[sl]);
      }
    }
    __syncthreads();  // the segment's entries read the scores stored above
  }
  uint64_t key[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = tid * R + r;
    uint64_t kv = ~uint64_t(0);
    if (i < len) {
      const int64_t slot = slot_r[r];
      // an out-of-range slot (rejected by the host) ranks below every real score
      const float sc = (slot >= 0 && slot < n_scores) ? scores[slot] : -INFINITY;
      kv = (uint64_t(orderable(sc)) << 32) | uint64_t(0xffffffffu - uint32_t(slot));
    }
    key[r] = kv;
  }

  int buf = 0;
  bitonic_sort<T, R, 2>(key, tid, xbuf, buf);

  // key[r] is now element tid * R + r of the ascending order
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = tid * R + r;
    if (i < len) {
      const int64_t slot = int64_t(0xffffffffu - uint32_t(key[r] & 0xffffffffu));
      slots[start + i] = slot;
      const int j = len - 1 - i;  // rank from the top
      if (topk_out && j < k) topk_out[int64_t(s) * k + j] = slot;
    }
  }
  if (topk_out) {
    for (int j = len + tid; j < k; j += T) topk_out[int64_t(s) * k + j] = -1;
  }
}

template <int T, int R>
hipError_t launch_rank(int64_t n_seg, hipStream_t st, const RankArgs& a) {
  if (a.part)
    hipLaunchKernelGGL((rank_kernel<T, R, true>), dim3(static_cast<unsigned>(n_seg)), dim3(T),
                       0, st, a);
  else
    hipLaunchKernelGGL((rank_kernel<T, R, false>), dim3(static_cast<unsigned>(n_seg)), dim3(T),
                       0, st, a);
  return hipGetLastError();
}

// Shared by both entry points: checks, then the launch shape by segment length.
int rank_entry(const char* fn, RankArgs a, int64_t n_seg, void* stream) {
  FDL_REQUIRE(n_seg >= 0 && n_seg < (int64_t(1) << 31), FDL_ERR_SHAPE,
              "%s: n_seg = %lld out of range", fn, (long long)n_seg);
  if (n_seg == 0) return ok();
  FDL_REQUIRE(a.scores && a.slots && a.seg, FDL_ERR_NULL, "%s: scores/slots/seg is NULL", fn);
  FDL_REQUIRE(a.max_len >= 0 && a.max_len <= kMaxLen, FDL_ERR_UNSUPPORTED,
              "%s: max_len = %d outside [0, %d]", fn, a.max_len, kMaxLen);
  FDL_REQUIRE(a.n_scores >= 1 && a.n_scores <= 0x7fffffff, FDL_ERR_SHAPE,
              "%s: n_scores = %lld outside [1, 2^31)", fn, (long long)a.n_scores);
  FDL_REQUIRE(a.k >= 0, FDL_ERR_SHAPE, "%s: k = %d < 0", fn, a.k);
  FDL_REQUIRE(a.topk_out != nullptr || a.k == 0, FDL_ERR_NULL,
              "%s: topk_out is NULL with k = %d", fn, a.k);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int m = a.max_len;
  hipError_t e;
  // One key per thread up to 1024 keys (threads rounded up to a power of two), then 2, 4 and
  // 8 keys per thread of 1024 threads. The segment is latency-bound: at 768 keys one key
  // per thread takes 6.5 us against 7.5 us at four keys per thread (measured on MI355X).
  if (m <= 64) e = launch_rank<64, 1>(n_seg, st, a);
  else if (m <= 128) e = launch_rank<128, 1>(n_seg, st, a);
  else if (m <= 256) e = launch_rank<256, 1>(n_seg, st, a);
  else if (m <= 512) e = launch_rank<512, 1>(n_seg, st, a);
  else if (m <= 1024) e = launch_rank<1024, 1>(n_seg, st, a);
  else if (m <= 2048) e = launch_rank<1024, 2>(n_seg, st, a);
  else if (m <= 4096) e = launch_rank<1024, 4>(n_seg, st, a);
  else e = launch_rank<1024, 8>(n_seg, st, a);
  FDL_HIP_CHECK(e);
  return ok();
}

}  // namespace
}  // namespace fdl

extern "C" int fdl_importance_rank(const float* scores, int64_t n_scores, int64_t* slots,
                                   int64_t n_slot_entries, const int32_t* seg, int64_t n_seg,
                                   int32_t max_len, int64_t* topk_out, int32_t k,
                                   void* stream) {
  fdl::RankArgs a{const_cast<float*>(scores), n_scores, slots, n_slot_entries, seg, max_len,
                  topk_out, k, nullptr, 0, 0.f, nullptr, 0, 0, 0, nullptr};
  return fdl::rank_entry("fdl_importance_rank", a, n_seg, stream);
}

extern "C" int fdl_importance_accumulate_rank(
    const float* imp_part, int64_t n_heads, float scale, const int32_t* page_table,
    int64_t n_seq, int64_t max_pages, int32_t page_log2, const int32_t* seg_keys, float* scores,
    int64_t n_scores, int64_t* slots, int64_t n_slot_entries, const int32_t* seg, int64_t n_seg,
    int32_t max_len, int64_t* topk_out, int32_t k, void* stream) {
  using namespace fdl;
  FDL_REQUIRE(n_heads >= 1 && n_heads <= 65535, FDL_ERR_SHAPE,
              "fdl_importance_accumulate_rank: n_heads = %lld outside [1, 65535]",
              (long long)n_heads);
  FDL_REQUIRE(n_seq >= 1 && n_seq < (int64_t(1) << 31) && max_pages >= 1 &&
                  max_pages < (int64_t(1) << 31),
              FDL_ERR_SHAPE, "fdl_importance_accumulate_rank: page table [%lld][%lld] out of range",
              (long long)n_seq, (long long)max_pages);
  FDL_REQUIRE(page_log2 >= 0 && page_log2 <= 16, FDL_ERR_SHAPE,
              "fdl_importance_accumulate_rank: page_log2 = %d outside [0, 16]", page_log2);
  FDL_REQUIRE(n_seg <= 0 || (imp_part && page_table && seg_keys), FDL_ERR_NULL,
              "fdl_importance_accumulate_rank: imp_part/page_table/seg_keys is NULL");
  RankArgs a{scores, n_scores, slots, n_slot_entries, seg, max_len, topk_out, k, imp_part,
             static_cast<int>(n_heads), scale, page_table, static_cast<int>(n_seq),
             static_cast<int>(max_pages), page_log2, seg_keys};
  return rank_entry("fdl_importance_accumulate_rank", a, n_seg, stream);
}
