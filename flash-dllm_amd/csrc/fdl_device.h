// Device-side helpers shared by the gfx950 kernels: vector types, bf16 conversion,
// 128-bit memory access and the bf16 MFMA wrappers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fdl {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

// 16-byte global load / store (the caller guarantees 16-byte alignment).
__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ u32x2 ld8(const void* p) {
  return *reinterpret_cast<const u32x2*>(p);
}
__device__ __forceinline__ void st8(void* p, u32x2 v) { *reinterpret_cast<u32x2*>(p) = v; }

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ bf16x8 as_bf16x8(u32x2 lo, u32x2 hi) {
  u32x4 v = {lo.x, lo.y, hi.x, hi.y};
  return __builtin_bit_cast(bf16x8, v);
}

// fp32 -> bf16, round to nearest even (the conversion torch's .to(torch.bfloat16) uses).
__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f2bf(lo)) | (static_cast<uint32_t>(f2bf(hi)) << 16);
}
__device__ __forceinline__ float bf2f(uint16_t h) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(h) << 16);
}

// fp32 -> fp16 pair (round to nearest even) as the bits of one 32-bit word, low half first;
// the bits of half `hi` of such a word back to fp32.
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(lo))) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(hi))) << 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t w, int hi) {
  return static_cast<float>(
      __builtin_bit_cast(_Float16, static_cast<uint16_t>(hi ? w >> 16 : w & 0xffffu)));
}

// D = A * B + C on one wavefront.
//   16x16x32: lane l supplies A[l % 16][8 * (l / 16) + j] and B[8 * (l / 16) + j][l % 16],
//             j = 0..7, and holds C[4 * (l / 16) + i][l % 16], i = 0..3.
//   32x32x16: lane l supplies A[l % 32][8 * (l / 32) + j] and B[8 * (l / 32) + j][l % 32],
//             and holds C[8 * (i / 4) + 4 * (l / 32) + i % 4][l % 32], i = 0..15.
// Within one instruction the reduction index is summed in full, so A and B may both use
// any one bijection between (lane group, j) and k.
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

}  // namespace fdl
