// Seeded synthetic fp16 weights: a counter-based standard normal that gives the same bits on the
// host (x86) and on gfx950. Element i of tensor (seed, tensor_id) is component (i & 1) of the
// Box-Muller pair j = i >> 1, whose two uniforms come from one splitmix64 output. Every float
// operation is an IEEE basic operation (+, -, *, /, sqrt, fma) in an explicit order, and this file
// is compiled with -ffp-contract=off, so both sides round identically; log, sin and cos are
// evaluated with fixed polynomials rather than library calls.
#include <algorithm>
#include <thread>
#include <vector>

#include "fw_common.h"

#define FW_HD __host__ __device__ __forceinline__

namespace fw {
namespace {

FW_HD uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

FW_HD uint32_t f32_bits(float f) {
  union {
    float f;
    uint32_t u;
  } c;
  c.f = f;
  return c.u;
}
FW_HD float bits_f32(uint32_t u) {
  union {
    float f;
    uint32_t u;
  } c;
  c.u = u;
  return c.f;
}

// Natural log for x in (0, 1): x = m * 2^e with m in [sqrt(1/2), sqrt(2)), ln m = 2 atanh(s),
// s = (m - 1) / (m + 1), odd series in s truncated after s^13 (|s| <= 0.1716).
FW_HD float synth_log(float x) {
  const uint32_t b = f32_bits(x);
  int e = static_cast<int>((b >> 23) & 0xFF) - 127;
  float m = bits_f32((b & 0x7FFFFFu) | 0x3F800000u);
  if (m > 1.41421356f) {
    m = m * 0.5f;
    e += 1;
  }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float s2 = s * s;
  float p = 1.0f / 13.0f;
  p = fmaf(p, s2, 1.0f / 11.0f);
  p = fmaf(p, s2, 1.0f / 9.0f);
  p = fmaf(p, s2, 1.0f / 7.0f);
  p = fmaf(p, s2, 1.0f / 5.0f);
  p = fmaf(p, s2, 1.0f / 3.0f);
  p = fmaf(p, s2, 1.0f);
  const float lnm = 2.0f * s * p;
  return fmaf(static_cast<float>(e), 0.693147180559945f, lnm);
}

// sin and cos of phi in [0, pi/2) by Taylor polynomials (truncation error < 1e-7).
FW_HD void synth_sincos(float phi, float* sn, float* cs) {
  const float x2 = phi * phi;
  float ps = -1.0f / 39916800.0f;
  ps = fmaf(ps, x2, 1.0f / 362880.0f);
  ps = fmaf(ps, x2, -1.0f / 5040.0f);
  ps = fmaf(ps, x2, 1.0f / 120.0f);
  ps = fmaf(ps, x2, -1.0f / 6.0f);
  ps = fmaf(ps, x2, 1.0f);
  *sn = phi * ps;
  float pc = 1.0f / 479001600.0f;
  pc = fmaf(pc, x2, -1.0f / 3628800.0f);
  pc = fmaf(pc, x2, 1.0f / 40320.0f);
  pc = fmaf(pc, x2, -1.0f / 720.0f);
  pc = fmaf(pc, x2, 1.0f / 24.0f);
  pc = fmaf(pc, x2, -0.5f);
  *cs = fmaf(pc, x2, 1.0f);
}

FW_HD float synth_normal(uint64_t key, uint64_t i) {
  const uint64_t h = mix64(key + ((i >> 1) + 1) * 0x9E3779B97F4A7C15ull);
  const uint32_t k1 = static_cast<uint32_t>(h >> 41);               // 23 bits
  const uint32_t k2 = static_cast<uint32_t>(h >> 9) & 0x7FFFFFu;    // 23 bits
  const float u1 = static_cast<float>(2u * k1 + 1u) * 5.9604644775390625e-8f;  // (2k+1) / 2^24, exact
  const float u2 = static_cast<float>(2u * k2 + 1u) * 5.9604644775390625e-8f;
  const float r = sqrtf(-2.0f * synth_log(u1));
  const float t = u2 * 4.0f;  // quadrant + fraction, exact
  const int q = static_cast<int>(t);
  const float phi = (t - static_cast<float>(q)) * 1.57079632679489662f;
  float sn, cs;
  synth_sincos(phi, &sn, &cs);
  float c, s;  // cos and sin of 2*pi*u2
  switch (q & 3) {
    case 0: c = cs; s = sn; break;
    case 1: c = -sn; s = cs; break;
    case 2: c = -cs; s = -sn; break;
    default: c = sn; s = -cs; break;
  }
  return r * ((i & 1) ? s : c);
}

FW_HD uint64_t synth_key(uint64_t seed, uint64_t tensor_id) {
  return mix64(mix64(seed + 0x9E3779B97F4A7C15ull) ^ (tensor_id * 0xD1B54A32D192ED03ull));
}

// fp32 -> binary16 bits, round to nearest even (host and device, no library dependence).
FW_HD uint16_t f32_to_f16_bits(float f) {
  const uint32_t x = f32_bits(f);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) return static_cast<uint16_t>(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
  if (ax >= 0x477FF000u) return static_cast<uint16_t>(sign | 0x7C00u);  // rounds to inf
  if (ax < 0x38800000u) {                                                // subnormal or zero in fp16
    if (ax < 0x33000000u) return static_cast<uint16_t>(sign);  // below 2^-25: rounds to zero
    // value = mant * 2^(E - 150) = v * 2^-24  =>  v = mant >> (126 - E), E in [102, 112].
    const uint32_t biased_e = ax >> 23;
    const uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
    const uint32_t sh = 126u - biased_e;
    uint32_t v = mant >> sh;
    const uint32_t rem = mant & ((1u << sh) - 1u);
    const uint32_t half = 1u << (sh - 1u);
    if (rem > half || (rem == half && (v & 1u))) ++v;
    return static_cast<uint16_t>(sign | v);
  }
  uint32_t v = ((ax - 0x38000000u) >> 13);
  const uint32_t rem = ax & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (v & 1u))) ++v;
  return static_cast<uint16_t>(sign | v);
}

__global__ void synth_kernel(uint16_t* dst, int64_t n, int64_t offset, uint64_t key, float mean, float sd) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float z = synth_normal(key, static_cast<uint64_t>(offset + i));
    dst[i] = f32_to_f16_bits(fmaf(sd, z, mean));
  }
}

}  // namespace
}  // namespace fw

extern "C" int fw_synth_normal_f16(void* dst, int64_t n, int64_t offset, uint64_t seed, uint64_t tensor_id,
                                   float mean, float std, hipStream_t stream) {
  if (!dst || n < 0 || offset < 0) return fw_fail(FW_EINVAL, "synth_normal_f16: bad arguments");
  if (n == 0) return FW_OK;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 65536);
  hipLaunchKernelGGL(fw::synth_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                     static_cast<uint16_t*>(dst), n, offset, fw::synth_key(seed, tensor_id), mean, std);
  return fw_check_launch("synth_normal_f16");
}

extern "C" int fw_synth_normal_f16_host(uint16_t* dst, int64_t n, int64_t offset, uint64_t seed, uint64_t tensor_id,
                                        float mean, float std) {
  if (!dst || n < 0 || offset < 0) return fw_fail(FW_EINVAL, "synth_normal_f16_host: bad arguments");
  const uint64_t key = fw::synth_key(seed, tensor_id);
  const int64_t kMinPerThread = 1 << 20;
  const int64_t hw = std::max<int64_t>(1, std::min<int64_t>(16, std::thread::hardware_concurrency()));
  const int64_t nt = std::max<int64_t>(1, std::min<int64_t>(hw, n / kMinPerThread));
  auto work = [=](int64_t lo, int64_t hi) {
    for (int64_t i = lo; i < hi; ++i)
      dst[i] = fw::f32_to_f16_bits(fmaf(std, fw::synth_normal(key, static_cast<uint64_t>(offset + i)), mean));
  };
  if (nt == 1) {
    work(0, n);
    return FW_OK;
  }
  std::vector<std::thread> threads;
  const int64_t per = (n + nt - 1) / nt;
  for (int64_t t = 0; t < nt; ++t) threads.emplace_back(work, t * per, std::min(n, (t + 1) * per));
  for (auto& th : threads) th.join();
  return FW_OK;
}
