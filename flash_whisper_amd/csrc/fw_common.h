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

// Butterfly steps between lane l and lane l ^ O without the LDS crossbar (a ds_bpermute costs an LDS
// round trip per step): O = 1, 2 are DPP quad permutes; O = 4, 8 are two DPP row shifts, each
// writing the 4-lane banks whose partner lies on its side; O = 16, 32 use v_permlane16_swap /
// v_permlane32_swap, which trade row pairs / wave halves between two copies of the value, so that
// the two results hold, lane by lane, the value and its partner. Every step combines the same two
// operands as a __shfl_xor step would.
template <int O>
__device__ __forceinline__ int xor_lane_bits(int x) {
  static_assert(O == 1 || O == 2 || O == 4 || O == 8, "DPP partner for O <= 8");
  int r;
  if constexpr (O == 1) {
    r = __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);  // quad_perm [1, 0, 3, 2]
  } else if constexpr (O == 2) {
    r = __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);  // quad_perm [2, 3, 0, 1]
  } else if constexpr (O == 4) {
    r = __builtin_amdgcn_update_dpp(0, x, 0x104, 0xF, 0x5, false);  // banks 0, 2 <- lane + 4 (row_shl:4)
    r = __builtin_amdgcn_update_dpp(r, x, 0x114, 0xF, 0xA, false);  // banks 1, 3 <- lane - 4 (row_shr:4)
  } else {
    r = __builtin_amdgcn_update_dpp(0, x, 0x108, 0xF, 0x3, false);  // banks 0, 1 <- lane + 8 (row_shl:8)
    r = __builtin_amdgcn_update_dpp(r, x, 0x118, 0xF, 0xC, false);  // banks 2, 3 <- lane - 8 (row_shr:8)
  }
  return r;
}
template <int O>
__device__ __forceinline__ float xor_lane(float v) {
  return __builtin_bit_cast(float, xor_lane_bits<O>(__builtin_bit_cast(int, v)));
}
// {v, v[l ^ O]} in some order per lane, for O = 16 or 32. Issued as inline assembly: the compiler's
// builtins for these swaps hand back the first register for both results. The leading s_nop covers
// the wait states a swap needs after the VALU write of its operands.
template <int O>
__device__ __forceinline__ void xor_pair(float v, float& a, float& b) {
  static_assert(O == 16 || O == 32, "row / half swaps");
  a = v;
  b = v;
  if constexpr (O == 16)
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  else
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
template <int O>
__device__ __forceinline__ float xor_add(float v) {
  if constexpr (O >= 16) {
    float a, b;
    xor_pair<O>(v, a, b);
    return a + b;
  } else {
    return v + xor_lane<O>(v);
  }
}
template <int O>
__device__ __forceinline__ float xor_max(float v) {
  if constexpr (O >= 16) {
    float a, b;
    xor_pair<O>(v, a, b);
    return fmaxf(a, b);
  } else {
    return fmaxf(v, xor_lane<O>(v));
  }
}

// Maximum of a 64-bit key over kWidth consecutive lanes (a power of two <= 64; every lane of the wave
// active) by the butterflies above, both halves of a key moved by the same exchange: no LDS round trips
// (a loop over keys in LDS, or ds_bpermute shuffles, costs one per step).
template <int O>
__device__ __forceinline__ unsigned long long u64_xor_max(unsigned long long v) {
  const int lo = static_cast<int>(static_cast<unsigned>(v)), hi = static_cast<int>(static_cast<unsigned>(v >> 32));
  unsigned long long a, b;
  if constexpr (O >= 16) {
    float alo, blo, ahi, bhi;
    xor_pair<O>(__builtin_bit_cast(float, lo), alo, blo);
    xor_pair<O>(__builtin_bit_cast(float, hi), ahi, bhi);
    a = (static_cast<unsigned long long>(__builtin_bit_cast(unsigned, ahi)) << 32) | __builtin_bit_cast(unsigned, alo);
    b = (static_cast<unsigned long long>(__builtin_bit_cast(unsigned, bhi)) << 32) | __builtin_bit_cast(unsigned, blo);
  } else {
    a = v;
    b = (static_cast<unsigned long long>(static_cast<unsigned>(xor_lane_bits<O>(hi))) << 32) |
        static_cast<unsigned>(xor_lane_bits<O>(lo));
  }
  return a > b ? a : b;
}
template <int kWidth>
__device__ __forceinline__ unsigned long long u64_group_max(unsigned long long v) {
  if constexpr (kWidth >= 64) v = u64_xor_max<32>(v);
  if constexpr (kWidth >= 32) v = u64_xor_max<16>(v);
  if constexpr (kWidth >= 16) v = u64_xor_max<8>(v);
  if constexpr (kWidth >= 8) v = u64_xor_max<4>(v);
  if constexpr (kWidth >= 4) v = u64_xor_max<2>(v);
  if constexpr (kWidth >= 2) v = u64_xor_max<1>(v);
  return v;
}

// Eight values per lane, a[t], each summed over the 8 lanes that share lane & 7 (partners lane ^ 8,
// then ^ 16, then ^ 32: the pairs and order of xor_add<32>(xor_add<16>(xor_add<8>(a[t])))), handing
// half of a lane's values to its partner at each step: 4 DPP exchanges, 2 row swaps and 1 half swap
// instead of 8 x 3 exchanges. Every add takes the same two operands as the butterfly's, so each sum is
// bit-identical to it. The lane ends with the sum of a[sum8_index(lane)].
__host__ __device__ constexpr int sum8_index(int lane) {
  return 4 * ((lane >> 3) & 1) + 2 * ((lane >> 4) & 1) + ((lane >> 5) & 1);
}
__device__ __forceinline__ float sum8_transposed(const float (&a)[8]) {
  const bool b3 = (threadIdx.x & 8) != 0;
  float r1[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    // lanes with bit 3 clear keep a[k] and take lane + 8's a[k]; the others keep a[k + 4] and take
    // lane - 8's a[k + 4] (two row shifts writing the banks of each side)
    int r = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, a[k]), 0x108, 0xF, 0x3, false);
    r = __builtin_amdgcn_update_dpp(r, __builtin_bit_cast(int, a[k + 4]), 0x118, 0xF, 0xC, false);
    r1[k] = (b3 ? a[k + 4] : a[k]) + __builtin_bit_cast(float, r);
  }
  // rows 0, 2 keep r1[m], rows 1, 3 r1[m + 2]: one row swap trades them, then one add
  float r2[2];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    float x = r1[m], y = r1[m + 2];
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(x), "+v"(y));
    r2[m] = x + y;
  }
  // lanes 0-31 keep r2[0], lanes 32-63 r2[1]
  float x = r2[0], y = r2[1];
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(x), "+v"(y));
  return x + y;
}

// Butterfly sum / max over `width` consecutive lanes (width a power of two <= 64), partners taken in
// the order width / 2, ..., 2, 1.
template <int kWidth>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (kWidth >= 64) v = xor_add<32>(v);
  if constexpr (kWidth >= 32) v = xor_add<16>(v);
  if constexpr (kWidth >= 16) v = xor_add<8>(v);
  if constexpr (kWidth >= 8) v = xor_add<4>(v);
  if constexpr (kWidth >= 4) v = xor_add<2>(v);
  if constexpr (kWidth >= 2) v = xor_add<1>(v);
  return v;
}
template <int kWidth>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (kWidth >= 64) v = xor_max<32>(v);
  if constexpr (kWidth >= 32) v = xor_max<16>(v);
  if constexpr (kWidth >= 16) v = xor_max<8>(v);
  if constexpr (kWidth >= 8) v = xor_max<4>(v);
  if constexpr (kWidth >= 4) v = xor_max<2>(v);
  if constexpr (kWidth >= 2) v = xor_max<1>(v);
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

// block_sum with the same arithmetic and one barrier: `red` is not reused before a later barrier, so the
// caller gives every reduction round its own kThreads/64 slots.
template <int kThreads>
__device__ __forceinline__ float block_sum_once(float v, float* red) {
  constexpr int kWaves = kThreads / kWave;
  v = group_sum<kWave>(v);
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) s += red[i];
  return s;
}

}  // namespace fw

// Records a launch error (if any) and returns the C-ABI status.
int fw_check_launch(const char* what);
int fw_fail(int code, const char* fmt, ...);
