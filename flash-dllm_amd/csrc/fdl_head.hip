// Confidence of the LM-head rows (gfx950): the float64 softmax maximum and its token, or
// the float64 softmax probability of a given token, one pass of reads per row.
//
// Replaces, for bf16 logits,
//   p = softmax(logits.to(float64), -1); x0_p, x0 = max(p, -1)        (generate.py:218, :320)
//   p = softmax(logits.to(float64), -1).gather(1, tok)                  (generate.py:337)
// For row r with maximum m (first index i_max):
//   s = sum_j exp(x_j - m) in float64; max probability = exp(0) / s = 1 / s;
//   probability of token t = exp(x_t - m) / s.
// A row with a NaN, a +inf or only -inf logits has a softmax of NaNs: probability NaN and
// index 0, as torch.max returns for it.
// bf16 -> float -> double is exact, so every term is the float64 softmax term; only the
// order of the float64 sum differs from torch's reduction.
#include <stdint.h>

#include "fdl_device.h"
#include "fdl_host.h"

namespace fdl {
namespace {

constexpr int kConfThreads = 256;  // one workgroup per row

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) {
  return __builtin_bit_cast(float, w & 0xffff0000u);
}

// (value, index) with the larger value, the smaller index among equal values.
__device__ __forceinline__ void arg_max_merge(float& m, int64_t& i, float m2, int64_t i2) {
  if (m2 > m || (m2 == m && i2 < i)) {
    m = m2;
    i = i2;
  }
}

// vocab % 8 == 0 and 16-byte aligned rows (checked on the host).
__global__ __launch_bounds__(kConfThreads) void softmax_conf_kernel(
    const uint16_t* __restrict__ logits, int64_t vocab, const int64_t* __restrict__ token,
    double* __restrict__ prob, int64_t* __restrict__ arg) {
  __shared__ float s_m[kConfThreads / kWave];
  __shared__ int64_t s_i[kConfThreads / kWave];
  __shared__ double s_sum[kConfThreads / kWave];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint16_t* x = logits + int64_t(blockIdx.x) * vocab;
  const int64_t n8 = vocab / 8;

  // pass 1: maximum and its first index (each thread visits increasing indices; a thread
  // that visits none keeps the index past every real one)
  float m = -INFINITY;
  int64_t im = INT64_MAX;
  for (int64_t c = tid; c < n8; c += kConfThreads) {
    const u32x4 v = ld16(x + 8 * c);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = bf16_lo(v[j]), b = bf16_hi(v[j]);
      if (a > m) {
        m = a;
        im = 8 * c + 2 * j;
      }
      if (b > m) {
        m = b;
        im = 8 * c + 2 * j + 1;
      }
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float m2 = __shfl_xor(m, off);
    const int64_t i2 = __shfl_xor(im, off);
    arg_max_merge(m, im, m2, i2);
  }
  if (lane == 0) {
    s_m[wave] = m;
    s_i[wave] = im;
  }
  __syncthreads();
  m = s_m[0];
  im = s_i[0];
#pragma unroll
  for (int w = 1; w < kConfThreads / kWave; ++w) arg_max_merge(m, im, s_m[w], s_i[w]);

  // pass 2: float64 sum of exp(x - m); per-thread partials, then a fixed reduction tree
  const double md = static_cast<double>(m);
  double s = 0.0;
  for (int64_t c = tid; c < n8; c += kConfThreads) {
    const u32x4 v = ld16(x + 8 * c);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s += exp(static_cast<double>(bf16_lo(v[j])) - md);
      s += exp(static_cast<double>(bf16_hi(v[j])) - md);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0) s_sum[wave] = s;
  __syncthreads();
  if (tid == 0) {
    double sum = s_sum[0];
#pragma unroll
    for (int w = 1; w < kConfThreads / kWave; ++w) sum += s_sum[w];
    double p;
    if (token) {
      const int64_t t = token[blockIdx.x];
      p = t >= 0 && t < vocab ? exp(static_cast<double>(bf2f(x[t])) - md) / sum : 0.0;
    } else {
      p = 1.0 / sum;
    }
    prob[blockIdx.x] = p;
    // A row with a NaN (no comparison above selects it, but it makes the sum NaN), a +inf or
    // only -inf logits has a softmax of NaNs; torch.max of it returns index 0.
    if (arg) arg[blockIdx.x] = __builtin_isfinite(m) && sum == sum ? im : 0;
  }
}

}  // namespace
}  // namespace fdl

extern "C" int fdl_softmax_confidence(const void* logits, int64_t n_rows, int64_t vocab,
                                      const int64_t* token, double* prob, int64_t* arg,
                                      void* stream) {
  using namespace fdl;
  FDL_REQUIRE(n_rows >= 0 && n_rows < (int64_t(1) << 31), FDL_ERR_SHAPE,
              "fdl_softmax_confidence: n_rows = %lld out of range", (long long)n_rows);
  FDL_REQUIRE(vocab >= 8 && vocab % 8 == 0, FDL_ERR_UNSUPPORTED,
              "fdl_softmax_confidence: vocab = %lld (a multiple of 8 is implemented)",
              (long long)vocab);
  if (n_rows == 0) return ok();
  FDL_REQUIRE_PTR(logits);
  FDL_REQUIRE_PTR(prob);
  FDL_REQUIRE_ALIGNED(logits, 16);
  hipLaunchKernelGGL(softmax_conf_kernel, dim3(static_cast<unsigned>(n_rows)),
                     dim3(kConfThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(logits), vocab, token, prob, arg);
  FDL_HIP_CHECK(hipGetLastError());
  return ok();
}
