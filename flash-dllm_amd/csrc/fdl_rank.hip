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
// whose ascending order is (score ascending, slot descending); the keys are bitonic-sorted
// in LDS (segment padded to a power of two with all-ones keys, which sort last).
#include "fdl_device.h"
#include "fdl_host.h"

namespace fdl {
namespace {

constexpr int kThreads = 1024;
constexpr int kMaxLen = 8192;

// Monotone map float -> uint32 (x < y  <=>  ord(x) < ord(y)); -0.0 and +0.0 map together.
__device__ __forceinline__ uint32_t orderable(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) == 0) u = 0;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__global__ __launch_bounds__(kThreads) void rank_kernel(const float* __restrict__ scores,
                                                        int64_t n_scores, int64_t* slots,
                                                        int64_t n_slot_entries,
                                                        const int32_t* __restrict__ seg,
                                                        int max_len, int64_t* topk_out, int k) {
  extern __shared__ uint64_t keys[];
  const int s = blockIdx.x;
  const int64_t start = seg[2 * s];
  int len = seg[2 * s + 1];
  // a segment longer than the LDS sized for max_len (rejected by the host) is left as is
  if (start < 0 || len < 0 || len > max_len || start + len > n_slot_entries) len = 0;
  int P = 1;
  while (P < len) P <<= 1;
  const int tid = threadIdx.x;
  for (int i = tid; i < P; i += kThreads) {
    uint64_t key = ~uint64_t(0);
    if (i < len) {
      const int64_t slot = slots[start + i];
      // an out-of-range slot (rejected by the host) ranks below every real score
      const float sc = (slot >= 0 && slot < n_scores) ? scores[slot] : -INFINITY;
      key = (uint64_t(orderable(sc)) << 32) | uint64_t(0xffffffffu - uint32_t(slot));
    }
    keys[i] = key;
  }
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      __syncthreads();
      for (int i = tid; i < (P >> 1); i += kThreads) {
        const int lo = 2 * stride * (i / stride) + (i % stride);
        const int hi = lo + stride;
        const bool up = (lo & size) == 0;
        const uint64_t x = keys[lo], y = keys[hi];
        if ((x > y) == up) {
          keys[lo] = y;
          keys[hi] = x;
        }
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < len; i += kThreads)
    slots[start + i] = int64_t(0xffffffffu - uint32_t(keys[i] & 0xffffffffu));
  if (topk_out) {
    for (int j = tid; j < k; j += kThreads) {
      topk_out[int64_t(s) * k + j] =
          j < len ? int64_t(0xffffffffu - uint32_t(keys[len - 1 - j] & 0xffffffffu)) : -1;
    }
  }
}

}  // namespace
}  // namespace fdl

extern "C" int fdl_importance_rank(const float* scores, int64_t n_scores, int64_t* slots,
                                   int64_t n_slot_entries, const int32_t* seg, int64_t n_seg,
                                   int32_t max_len, int64_t* topk_out, int32_t k,
                                   void* stream) {
  using namespace fdl;
  FDL_REQUIRE(n_seg >= 0 && n_seg < (int64_t(1) << 31), FDL_ERR_SHAPE,
              "fdl_importance_rank: n_seg = %lld out of range", (long long)n_seg);
  if (n_seg == 0) return ok();
  FDL_REQUIRE_PTR(scores);
  FDL_REQUIRE_PTR(slots);
  FDL_REQUIRE_PTR(seg);
  FDL_REQUIRE(max_len >= 0 && max_len <= kMaxLen, FDL_ERR_UNSUPPORTED,
              "fdl_importance_rank: max_len = %d outside [0, %d]", max_len, kMaxLen);
  FDL_REQUIRE(n_scores >= 1 && n_scores <= 0x7fffffff, FDL_ERR_SHAPE,
              "fdl_importance_rank: n_scores = %lld outside [1, 2^31)", (long long)n_scores);
  FDL_REQUIRE(k >= 0, FDL_ERR_SHAPE, "fdl_importance_rank: k = %d < 0", k);
  FDL_REQUIRE(topk_out != nullptr || k == 0, FDL_ERR_NULL,
              "fdl_importance_rank: topk_out is NULL with k = %d", k);
  int P = 1;
  while (P < max_len) P <<= 1;
  const size_t lds = sizeof(uint64_t) * static_cast<size_t>(P);
  hipLaunchKernelGGL(rank_kernel, dim3(static_cast<unsigned>(n_seg)), dim3(kThreads), lds,
                     static_cast<hipStream_t>(stream), scores, n_scores, slots, n_slot_entries,
                     seg, max_len, topk_out, k);
  FDL_HIP_CHECK(hipGetLastError());
  return ok();
}
