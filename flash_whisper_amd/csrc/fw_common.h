// Shared device helpers for the flash_whisper_amd kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/flash_whisper.h"

namespace fw {

constexpr int kWave = 64;         // CDNA wavefront width
constexpr int kHidden = 1280;     // whisper-large-v3-turbo d_model
constexpr int kHeadDim = 64;      // d_model / heads
constexpr int kSplitKeys = 64;    // keys per split block (reference kSplitKeys)

typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef _Float16 h4v __attribute__((ext_vector_type(4)));
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));

// 16-byte aligned bundle of 8 halves, loaded with one global_load_dwordx4.
struct __align__(16) H8 {
  uint4 u;
};

__device__ __forceinline__ float h2f(_Float16 x) { return static_cast<float>(x); }
__device__ __forceinline__ _Float16 f2h(float x) { return static_cast<_Float16>(x); }  // round-to-nearest-even
__device__ __forceinline__ float round_h(float x) { return static_cast<float>(static_cast<_Float16>(x)); }

// Butterfly sum over `width` consecutive lanes (width a power of two <= 64).
template <int kWidth>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = kWidth / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
template <int kWidth>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = kWidth / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Dot of 8 fp16 pairs accumulated in fp32 with v_dot2_f32_f16.
__device__ __forceinline__ float dot8(const uint4& a, const uint4& b, float acc) {
  const h2v* pa = reinterpret_cast<const h2v*>(&a);
  const h2v* pb = reinterpret_cast<const h2v*>(&b);
#pragma unroll
  for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_fdot2(pa[i], pb[i], acc, false);
  return acc;
}

// Non-temporal 16-byte load for streamed-once weights.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Orders (value, index) so a larger u64 means a larger value, ties going to the lower index
// (the same order as torch.argmax). Zero means "no candidate".
__device__ __forceinline__ unsigned long long pack_score(float v, int idx) {
  unsigned int u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (static_cast<unsigned long long>(u) << 32) | (0xFFFFFFFFu - static_cast<unsigned int>(idx));
}

// Exact-erf GELU as torch's F.gelu default: 0.5 * x * (1 + erf(x / sqrt(2))).
__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

// Block-wide sum for a block of kThreads threads; `red` must hold kThreads/64 floats.
template <int kThreads>
__device__ __forceinline__ float block_sum(float v, float* red) {
  constexpr int kWaves = kThreads / kWave;
  v = group_sum<kWave>(v);
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) s += red[i];
  __syncthreads();
  return s;
}

}  // namespace fw

// Records a launch error (if any) and returns the C-ABI status.
int fw_check_launch(const char* what);
int fw_fail(int code, const char* fmt, ...);
