// Elementwise parts of the transformer block around the Flash-Cache path, fused so that
// each is one pass over HBM (gfx950).
//
//  * fdl_rms_norm: the RMSLayerNorm that produces the projection input
//    (flash_cache_triton.py:494, modeling_llada.py:389-403) and, with a residual, the
//    attention residual add followed by ff_norm (flash_cache_triton.py:618-624):
//        s   = bf16(x + r)                      (when r is given; written to sum_out)
//        y   = bf16(s * rsqrt(mean(s^2) + eps)) (fp32 statistics)
//        out = bf16(weight * y)
//  * fdl_silu_mul: act(ff_proj(x)) * up_proj(x) (flash_cache_triton.py:628-633) with the
//    SiLU activation: out = bf16(bf16(silu(g)) * u).
// The roundings to bf16 sit where the unfused PyTorch code rounds.
#include "fdl_device.h"
#include "fdl_host.h"

namespace fdl {
namespace {

constexpr int kNormThreads = 256;  // one workgroup per row

__device__ __forceinline__ float bf_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) {
  return __builtin_bit_cast(float, w & 0xffff0000u);
}
__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

// Row r: chunks of 8 bf16 strided by the workgroup; d % 8 == 0 (checked on the host).
template <bool kResidual>
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ res,
    const uint16_t* __restrict__ w, int d, float eps, uint16_t* __restrict__ sum_out,
    uint16_t* __restrict__ out) {
  constexpr int kMaxChunks = 4;  // d <= 8 * 256 * 4 = 8192
  __shared__ float red[kNormThreads / kWave];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int n_chunks = d / 8;
  const uint16_t* xr = x + row * d;
  u32x4 v[kMaxChunks];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const int c = tid + kNormThreads * i;
    if (c < n_chunks) {
      u32x4 a = ld16(xr + 8 * c);
      if constexpr (kResidual) {
        const u32x4 b = ld16(res + row * d + 8 * c);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          a[j] = pack_bf16x2(bf_lo(a[j]) + bf_lo(b[j]), bf_hi(a[j]) + bf_hi(b[j]));
        st16(sum_out + row * d + 8 * c, a);
      }
      v[i] = a;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = bf_lo(a[j]), hi = bf_hi(a[j]);
        ss += lo * lo + hi * hi;
      }
    }
  }
  // workgroup sum of squares
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / kWave; ++i) tot += red[i];
  const float inv = 1.0f / sqrtf(tot / float(d) + eps);
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const int c = tid + kNormThreads * i;
    if (c < n_chunks) {
      const u32x4 wv = ld16(w + 8 * c);
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float ylo = round_bf(bf_lo(v[i][j]) * inv), yhi = round_bf(bf_hi(v[i][j]) * inv);
        o[j] = pack_bf16x2(bf_lo(wv[j]) * ylo, bf_hi(wv[j]) * yhi);
      }
      st16(out + row * d + 8 * c, o);
    }
  }
}

constexpr int kEwThreads = 256;

__global__ __launch_bounds__(kEwThreads) void silu_mul_kernel(const uint16_t* __restrict__ g,
                                                              const uint16_t* __restrict__ u,
                                                              int64_t n8,
                                                              uint16_t* __restrict__ out) {
  for (int64_t c = int64_t(blockIdx.x) * kEwThreads + threadIdx.x; c < n8;
       c += int64_t(gridDim.x) * kEwThreads) {
    const u32x4 a = ld16(g + 8 * c), b = ld16(u + 8 * c);
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float g0 = bf_lo(a[j]), g1 = bf_hi(a[j]);
      const float s0 = round_bf(g0 / (1.0f + expf(-g0)));
      const float s1 = round_bf(g1 / (1.0f + expf(-g1)));
      o[j] = pack_bf16x2(s0 * bf_lo(b[j]), s1 * bf_hi(b[j]));
    }
    st16(out + 8 * c, o);
  }
}

// Rows of a [gate | up] buffer: row r's gate at g + r * ld, its up at u + r * ld. The
// output row is cut into column chunks of q8 16-byte vectors (w8 = n_chunks * q8 per row);
// chunk q of row r goes to out + 8 * (q * n_rows * q8 + r * q8) (one chunk: plain rows).
__global__ __launch_bounds__(kEwThreads) void silu_mul_rows_kernel(
    const uint16_t* __restrict__ g, const uint16_t* __restrict__ u, int64_t ld, int64_t w8,
    int64_t q8, int64_t n_rows, int64_t n8, uint16_t* __restrict__ out) {
  for (int64_t c = int64_t(blockIdx.x) * kEwThreads + threadIdx.x; c < n8;
       c += int64_t(gridDim.x) * kEwThreads) {
    const int64_t r = c / w8, j8 = c - r * w8;
    const int64_t q = j8 / q8;
    const int64_t o8 = (q * n_rows + r) * q8 + (j8 - q * q8);
    const u32x4 a = ld16(g + r * ld + 8 * j8), b = ld16(u + r * ld + 8 * j8);
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float g0 = bf_lo(a[j]), g1 = bf_hi(a[j]);
      const float s0 = round_bf(g0 / (1.0f + expf(-g0)));
      const float s1 = round_bf(g1 / (1.0f + expf(-g1)));
      o[j] = pack_bf16x2(s0 * bf_lo(b[j]), s1 * bf_hi(b[j]));
    }
    st16(out + 8 * o8, o);
  }
}

// out[i] = bf16(float(out[i]) + sum_s part[s][i]), the partials summed in ascending s first;
// 8 columns (one 16-byte bf16 vector, two 16-byte fp32 vectors per partial) per step.
__global__ __launch_bounds__(kEwThreads) void split_reduce_residual_kernel(
    const float* __restrict__ part, int n_split, int64_t stride, int64_t n8,
    uint16_t* __restrict__ out) {
  for (int64_t c = int64_t(blockIdx.x) * kEwThreads + threadIdx.x; c < n8;
       c += int64_t(gridDim.x) * kEwThreads) {
    float acc[8];
    {
      const f32x4 a = *reinterpret_cast<const f32x4*>(part + 8 * c);
      const f32x4 b = *reinterpret_cast<const f32x4*>(part + 8 * c + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[j] = a[j];
        acc[4 + j] = b[j];
      }
    }
    for (int sp = 1; sp < n_split; ++sp) {
      const float* p = part + sp * stride + 8 * c;
      const f32x4 a = *reinterpret_cast<const f32x4*>(p);
      const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[j] += a[j];
        acc[4 + j] += b[j];
      }
    }
    const u32x4 r = ld16(out + 8 * c);
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = pack_bf16x2(bf_lo(r[j]) + acc[2 * j], bf_hi(r[j]) + acc[2 * j + 1]);
    st16(out + 8 * c, o);
  }
}

}  // namespace
}  // namespace fdl

extern "C" int fdl_rms_norm(const void* x, const void* residual, const void* weight,
                            int64_t n_rows, int64_t d, float eps, void* sum_out, void* out,
                            void* stream) {
  using namespace fdl;
  FDL_REQUIRE(n_rows >= 0 && n_rows < (int64_t(1) << 31), FDL_ERR_SHAPE,
              "fdl_rms_norm: n_rows = %lld out of range", (long long)n_rows);
  FDL_REQUIRE(d >= 8 && d <= 8192 && d % 8 == 0, FDL_ERR_UNSUPPORTED,
              "fdl_rms_norm: d = %lld (a multiple of 8 up to 8192 is implemented)",
              (long long)d);
  FDL_REQUIRE(eps >= 0.f, FDL_ERR_SHAPE, "fdl_rms_norm: eps < 0");
  if (n_rows == 0) return ok();
  FDL_REQUIRE_PTR(x);
  FDL_REQUIRE_PTR(weight);
  FDL_REQUIRE_PTR(out);
  FDL_REQUIRE(residual == nullptr || sum_out != nullptr, FDL_ERR_NULL,
              "fdl_rms_norm: sum_out is NULL with a residual");
  FDL_REQUIRE_ALIGNED(x, 16);
  FDL_REQUIRE_ALIGNED(weight, 16);
  FDL_REQUIRE_ALIGNED(out, 16);
  if (residual) {
    FDL_REQUIRE_ALIGNED(residual, 16);
    FDL_REQUIRE_ALIGNED(sum_out, 16);
  }
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const auto* xp = static_cast<const uint16_t*>(x);
  const auto* rp = static_cast<const uint16_t*>(residual);
  const auto* wp = static_cast<const uint16_t*>(weight);
  auto* sp = static_cast<uint16_t*>(sum_out);
  auto* op = static_cast<uint16_t*>(out);
  if (residual)
    hipLaunchKernelGGL(rms_norm_kernel<true>, dim3(static_cast<unsigned>(n_rows)),
                       dim3(kNormThreads), 0, st, xp, rp, wp, static_cast<int>(d), eps, sp, op);
  else
    hipLaunchKernelGGL(rms_norm_kernel<false>, dim3(static_cast<unsigned>(n_rows)),
                       dim3(kNormThreads), 0, st, xp, rp, wp, static_cast<int>(d), eps, sp, op);
  FDL_HIP_CHECK(hipGetLastError());
  return ok();
}

extern "C" int fdl_silu_mul(const void* gate, const void* up, int64_t n, void* out,
                            void* stream) {
  using namespace fdl;
  FDL_REQUIRE(n >= 0 && n % 8 == 0, FDL_ERR_UNSUPPORTED,
              "fdl_silu_mul: n = %lld (a multiple of 8 is implemented)", (long long)n);
  if (n == 0) return ok();
  FDL_REQUIRE_PTR(gate);
  FDL_REQUIRE_PTR(up);
  FDL_REQUIRE_PTR(out);
  FDL_REQUIRE_ALIGNED(gate, 16);
  FDL_REQUIRE_ALIGNED(up, 16);
  FDL_REQUIRE_ALIGNED(out, 16);
  const int64_t n8 = n / 8;
  const int64_t blocks = std::min<int64_t>((n8 + kEwThreads - 1) / kEwThreads, 256 * 8);
  hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kEwThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(gate),
                     static_cast<const uint16_t*>(up), n8, static_cast<uint16_t*>(out));
  FDL_HIP_CHECK(hipGetLastError());
  return ok();
}

extern "C" int fdl_silu_mul_rows(const void* gate, const void* up, int64_t n_rows,
                                 int64_t width, int64_t ld, int64_t out_chunks, void* out,
                                 void* stream) {
  using namespace fdl;
  FDL_REQUIRE(n_rows >= 0 && width >= 0 && width % 8 == 0 && ld % 8 == 0 && ld >= width,
              FDL_ERR_UNSUPPORTED,
              "fdl_silu_mul_rows: width = %lld, ld = %lld (multiples of 8, ld >= width)",
              (long long)width, (long long)ld);
  FDL_REQUIRE(out_chunks >= 1 && width % (8 * out_chunks) == 0, FDL_ERR_UNSUPPORTED,
              "fdl_silu_mul_rows: out_chunks = %lld must divide width / 8 = %lld",
              (long long)out_chunks, (long long)(width / 8));
  if (n_rows == 0 || width == 0) return ok();
  FDL_REQUIRE_PTR(gate);
  FDL_REQUIRE_PTR(up);
  FDL_REQUIRE_PTR(out);
  FDL_REQUIRE_ALIGNED(gate, 16);
  FDL_REQUIRE_ALIGNED(up, 16);
  FDL_REQUIRE_ALIGNED(out, 16);
  const int64_t w8 = width / 8, n8 = n_rows * w8;
  const int64_t blocks = std::min<int64_t>((n8 + kEwThreads - 1) / kEwThreads, 256 * 8);
  hipLaunchKernelGGL(silu_mul_rows_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kEwThreads),
                     0, static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(gate),
                     static_cast<const uint16_t*>(up), ld, w8, w8 / out_chunks, n_rows, n8,
                     static_cast<uint16_t*>(out));
  FDL_HIP_CHECK(hipGetLastError());
  return ok();
}

extern "C" int fdl_split_reduce_residual(const float* part, int64_t n_split, int64_t n_rows,
                                         int64_t n_cols, void* residual_out, void* stream) {
  using namespace fdl;
  FDL_REQUIRE(n_split >= 1 && n_split <= 64, FDL_ERR_UNSUPPORTED,
              "fdl_split_reduce_residual: n_split = %lld outside [1, 64]", (long long)n_split);
  FDL_REQUIRE(n_rows >= 0 && n_cols >= 0 && n_cols % 8 == 0, FDL_ERR_UNSUPPORTED,
              "fdl_split_reduce_residual: n_cols = %lld (a multiple of 8 is implemented)",
              (long long)n_cols);
  if (n_rows == 0 || n_cols == 0) return ok();
  FDL_REQUIRE_PTR(part);
  FDL_REQUIRE_PTR(residual_out);
  FDL_REQUIRE_ALIGNED(part, 16);
  FDL_REQUIRE_ALIGNED(residual_out, 16);
  const int64_t n = n_rows * n_cols, n8 = n / 8;
  const int64_t blocks = std::min<int64_t>((n8 + kEwThreads - 1) / kEwThreads, 256 * 8);
  hipLaunchKernelGGL(split_reduce_residual_kernel, dim3(static_cast<unsigned>(blocks)),
                     dim3(kEwThreads), 0, static_cast<hipStream_t>(stream), part,
                     static_cast<int>(n_split), n, n8, static_cast<uint16_t*>(residual_out));
  FDL_HIP_CHECK(hipGetLastError());
  return ok();
}
