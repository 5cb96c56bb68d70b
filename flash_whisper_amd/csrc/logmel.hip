// Log-mel front end for gfx950 (replaces the torch.stft path of custom/model.py:93-98, whose
// arithmetic is WhisperFeatureExtractor._torch_extract_fbank_features):
//   frames: centred STFT, n_fft = 400, hop = 160, periodic Hann, reflect padding, last frame dropped
//   power:  |X[k]|^2 for the 201 one-sided bins
//   mel:    filters^T (128 x 201) @ power, log10(max(., 1e-10))
//   final:  max(x, global_max - 8), (x + 4) / 4
// Prepare (one block, once per filterbank): the twiddle table exp(-2 pi i n / 400) built in fp64, and
// the compacted filterbank (each mel's triangle is a short run of bins: its first bin, the run length
// and the run's weights). Frames (one block per 12 frames): stages the reflect-padded samples in LDS,
// applies the window, and takes each frame's 400-point real DFT as a 200-point complex FFT of the
// (even, odd) sample pairs (Stockham autosort, radices 8, 5, 5, natural order out) followed by the
// real-input split; then the power, the compacted filterbank (the same terms in the same order as the
// dense product, whose other terms are zero), log10 and one block maximum. Finalize reduces the block
// maxima, clamps, rescales and writes the fp16 time-major copy the encoder's conv stem reads.
#include <algorithm>
#include <cstring>
#include "fw_common.h"

namespace fw {
namespace {

constexpr int kNfft = 400, kHop = 160, kBins = 201, kMels = 128;
constexpr int kHalf = kNfft / 2;  // complex FFT length
constexpr int kFramesPerBlock = 12;
constexpr int kSpan = (kFramesPerBlock - 1) * kHop + kNfft;  // samples staged per block
constexpr int kRun = 16;  // longest compacted filter run; longer ones are read from the dense filters
// Workspace layout (floats): the twiddles (float2 x 400), per mel {first bin, run length} (int2 x 128),
// per mel kRun weights, then one maximum per frames block. The prepared part does not depend on the
// number of samples.
constexpr int kWsTw = 0, kWsRange = kWsTw + 2 * kNfft, kWsW = kWsRange + 2 * kMels, kWsMax = kWsW + kMels * kRun;
static_assert(kWsRange % 2 == 0 && kWsMax % 4 == 0, "float2 / int2 / 16-byte alignment of the workspace parts");

__global__ void __launch_bounds__(1024) logmel_prepare_kernel(const float* __restrict__ filters, float* __restrict__ ws) {
  const int tid = threadIdx.x;
  if (tid < kNfft) {  // exp(-2 pi i n / 400)
    double sn, cs;
    sincospi(static_cast<double>(tid) / 200.0, &sn, &cs);
    reinterpret_cast<float2*>(ws + kWsTw)[tid] = make_float2(static_cast<float>(cs), static_cast<float>(-sn));
  }
  // Eight lanes per mel (in one wave), each scanning a slice of the bins for the first and last nonzero.
  constexpr int kSlice = (kBins + 7) / 8;
  const int m = tid >> 3, part = tid & 7;
  float v[kSlice];
#pragma unroll
  for (int i = 0; i < kSlice; ++i) {
    const int k = part * kSlice + i;
    v[i] = k < kBins ? filters[k * kMels + m] : 0.f;
  }
  int lo = kBins, hi = -1;
#pragma unroll
  for (int i = 0; i < kSlice; ++i) {
    const int k = part * kSlice + i;
    if (v[i] != 0.f) {
      lo = min(lo, k);
      hi = max(hi, k);
    }
  }
#pragma unroll
  for (int o = 1; o < 8; o <<= 1) {
    lo = min(lo, __shfl_xor(lo, o));
    hi = max(hi, __shfl_xor(hi, o));
  }
  const int len = hi < 0 ? 0 : hi - lo + 1;
  const int first = hi < 0 ? 0 : lo;
  if (part == 0) reinterpret_cast<int2*>(ws + kWsRange)[m] = make_int2(first, len);
  float* w = ws + kWsW;
  for (int j = part; j < kRun; j += 8) w[m * kRun + j] = (j < len && len <= kRun) ? filters[(first + j) * kMels + m] : 0.f;
}

// torch.stft reflect padding (valid for |overhang| < n). Samples staged for frames past the last one
// can overhang further; they are never used, so the index is only clamped into the buffer.
__device__ __forceinline__ int reflect(int i, int n) {
  if (i < 0) i = -i;
  if (i >= n) i = 2 * (n - 1) - i;
  return i < 0 ? 0 : (i >= n ? n - 1 : i);
}

__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
  return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
__device__ __forceinline__ float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }
__device__ __forceinline__ float2 mul_mi(float2 a) { return make_float2(a.y, -a.x); }  // -i a

// In-register DFTs with the forward sign, V[b] = sum_a v[a] exp(-2 pi i a b / R).
__device__ __forceinline__ void dft4(float2& a0, float2& a1, float2& a2, float2& a3) {
  const float2 s0 = cadd(a0, a2), d0 = csub(a0, a2), s1 = cadd(a1, a3), d1 = mul_mi(csub(a1, a3));
  a0 = cadd(s0, s1);
  a2 = csub(s0, s1);
  a1 = cadd(d0, d1);
  a3 = csub(d0, d1);
}
__device__ __forceinline__ void dft8(float2 (&v)[8]) {
  // even / odd halves, then the W8^k combination
  dft4(v[0], v[2], v[4], v[6]);
  dft4(v[1], v[3], v[5], v[7]);
  constexpr float r = 0.70710678118654752f;
  const float2 o0 = v[1], o1 = cmul(v[3], make_float2(r, -r)), o2 = mul_mi(v[5]), o3 = cmul(v[7], make_float2(-r, -r));
  const float2 e0 = v[0], e1 = v[2], e2 = v[4], e3 = v[6];
  v[0] = cadd(e0, o0);
  v[4] = csub(e0, o0);
  v[1] = cadd(e1, o1);
  v[5] = csub(e1, o1);
  v[2] = cadd(e2, o2);
  v[6] = csub(e2, o2);
  v[3] = cadd(e3, o3);
  v[7] = csub(e3, o3);
}
__device__ __forceinline__ void dft5(float2 (&v)[5]) {
  constexpr float c1 = 0.30901699437494742f, c2 = -0.80901699437494742f;  // cos(2 pi / 5), cos(4 pi / 5)
  constexpr float s1 = 0.95105651629515357f, s2 = 0.58778525229247313f;   // sin(2 pi / 5), sin(4 pi / 5)
  const float2 t1 = cadd(v[1], v[4]), t2 = cadd(v[2], v[3]), t3 = csub(v[1], v[4]), t4 = csub(v[2], v[3]);
  const float2 a1 = make_float2(v[0].x + c1 * t1.x + c2 * t2.x, v[0].y + c1 * t1.y + c2 * t2.y);
  const float2 a2 = make_float2(v[0].x + c2 * t1.x + c1 * t2.x, v[0].y + c2 * t1.y + c1 * t2.y);
  const float2 b1 = make_float2(s1 * t3.x + s2 * t4.x, s1 * t3.y + s2 * t4.y);
  const float2 b2 = make_float2(s2 * t3.x - s1 * t4.x, s2 * t3.y - s1 * t4.y);
  v[0] = cadd(v[0], cadd(t1, t2));
  v[1] = cadd(a1, mul_mi(b1));
  v[4] = csub(a1, mul_mi(b1));
  v[2] = cadd(a2, mul_mi(b2));
  v[3] = csub(a2, mul_mi(b2));
}
template <int R>
__device__ __forceinline__ void dft(float2 (&v)[R]) {
  if constexpr (R == 8) dft8(v);
  else dft5(v);
}

// One Stockham stage of the 200-point FFT for every frame of the block: butterfly j of a frame reads
// src[j + r * 200 / R], applies the twiddles exp(-2 pi i (j mod NS) r / (NS R)) (table index
// (j mod NS) r 400 / (NS R) < 400), runs the radix-R DFT and writes dst[(j / NS) NS R + j mod NS + r NS].
template <int R, int NS>
__device__ __forceinline__ void fft_stage(const float2 (*src)[kHalf], float2 (*dst)[kHalf], const float2* tw, int tid) {
  constexpr int kB = kHalf / R, kStep = kNfft / (NS * R);
  static_assert(kHalf % R == 0 && kNfft % (NS * R) == 0 && (NS - 1) * (R - 1) * kStep < kNfft, "stage shape");
  for (int i = tid; i < kFramesPerBlock * kB; i += 256) {
    const int f = i / kB, j = i - f * kB;
    float2 v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = src[f][j + r * kB];
    if constexpr (NS > 1) {
      const int a = (j % NS) * kStep;
#pragma unroll
      for (int r = 1; r < R; ++r) v[r] = cmul(v[r], tw[a * r]);
    }
    dft<R>(v);
    const int base = (j / NS) * NS * R + j % NS;
#pragma unroll
    for (int r = 0; r < R; ++r) dst[f][base + r * NS] = v[r];
  }
}

__global__ void __launch_bounds__(256) logmel_frames_kernel(const float* __restrict__ wave, int n_samples,
                                                            int n_frames, const float* __restrict__ filters,
                                                            const float* __restrict__ ws, float* __restrict__ out,
                                                            float* __restrict__ block_max) {
  __shared__ float xs[kSpan];
  __shared__ float2 tw[kNfft];
  __shared__ float2 za[kFramesPerBlock][kHalf];
  __shared__ float2 zb[kFramesPerBlock][kHalf];
  __shared__ __align__(16) float pw[kBins][kFramesPerBlock];
  __shared__ int2 mrange[kMels];
  __shared__ float mw[kMels * kRun];
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int f0 = blockIdx.x * kFramesPerBlock;
  const int s0 = f0 * kHop - kNfft / 2;

  for (int i = tid; i < kSpan; i += 256) xs[i] = wave[reflect(s0 + i, n_samples)];
  for (int i = tid; i < kNfft; i += 256) tw[i] = reinterpret_cast<const float2*>(ws + kWsTw)[i];
  if (tid < kMels) mrange[tid] = reinterpret_cast<const int2*>(ws + kWsRange)[tid];
  for (int i = tid; i < kMels * kRun; i += 256) mw[i] = ws[kWsW + i];
  __syncthreads();
  // z[m] = (x[2m], x[2m + 1]) windowed; periodic Hann 0.5 - 0.5 cos(2 pi n / 400)
  for (int i = tid; i < kFramesPerBlock * kHalf; i += 256) {
    const int f = i / kHalf, m = i - f * kHalf, n = 2 * m;
    const float w0 = 0.5f - 0.5f * tw[n].x, w1 = 0.5f - 0.5f * tw[n + 1].x;
    za[f][m] = make_float2(xs[f * kHop + n] * w0, xs[f * kHop + n + 1] * w1);
  }
  __syncthreads();
  fft_stage<8, 1>(za, zb, tw, tid);
  __syncthreads();
  fft_stage<5, 8>(zb, za, tw, tid);
  __syncthreads();
  fft_stage<5, 40>(za, zb, tw, tid);
  __syncthreads();
  // X[k] = E[k] + exp(-2 pi i k / 400) O[k] with E = (Z[k] + conj Z[200 - k]) / 2 and
  // O = (Z[k] - conj Z[200 - k]) / 2i, indices mod 200; power |X[k]|^2.
  for (int i = tid; i < kFramesPerBlock * kBins; i += 256) {
    const int f = i / kBins, k = i - f * kBins;
    const float2 zk = zb[f][k % kHalf], zc = zb[f][(kHalf - k) % kHalf];
    const float2 e = make_float2(0.5f * (zk.x + zc.x), 0.5f * (zk.y - zc.y));
    const float2 o = make_float2(0.5f * (zk.y + zc.y), -0.5f * (zk.x - zc.x));
    const float2 x = cadd(e, cmul(tw[k], o));
    pw[k][f] = x.x * x.x + x.y * x.y;
  }
  __syncthreads();

  // filterbank: the nonzero terms of filters^T @ power in increasing bin order, as the dense sum
  constexpr int kF = kFramesPerBlock / 2;  // 2 groups of frames per mel
  const int m = tid & (kMels - 1), fh = tid >> 7;
  float acc[kF];
#pragma unroll
  for (int f = 0; f < kF; ++f) acc[f] = 0.f;
  const int2 rg = mrange[m];
  for (int j = 0; j < rg.y; ++j) {
    const int k = rg.x + j;
    const float fk = rg.y <= kRun ? mw[m * kRun + j] : filters[k * kMels + m];
    if (fk != 0.f) {
#pragma unroll
      for (int f = 0; f < kF; ++f) acc[f] = fmaf(fk, pw[k][fh * kF + f], acc[f]);
    }
  }
  float vmax = -INFINITY;
#pragma unroll
  for (int f = 0; f < kF; ++f) {
    const int t = f0 + fh * kF + f;
    if (t < n_frames) {
      const float v = log10f(fmaxf(acc[f], 1e-10f));
      out[static_cast<size_t>(m) * n_frames + t] = v;
      vmax = fmaxf(vmax, v);
    }
  }
  vmax = group_max<kWave>(vmax);
  if ((tid & 63) == 0) red[tid >> 6] = vmax;
  __syncthreads();
  if (tid == 0) block_max[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

constexpr int kTileT = 16;                     // frames per finalize block
constexpr int kFinPer = kMels * kTileT / 256;  // values per thread

__global__ void __launch_bounds__(256) logmel_finalize_kernel(float* __restrict__ out, _Float16* __restrict__ out16,
                                                              int n_frames, const float* __restrict__ block_max,
                                                              int n_blocks) {
  __shared__ float red[4];
  __shared__ _Float16 tile[kTileT][kMels + 2];
  const int tid = threadIdx.x;
  const int t0 = blockIdx.x * kTileT;
  // this block's values are requested before the block maxima are reduced
  float v[kFinPer];
#pragma unroll
  for (int q = 0; q < kFinPer; ++q) {
    const int i = tid + 256 * q, mm = i / kTileT, t = t0 + i % kTileT;
    v[q] = t < n_frames ? out[static_cast<size_t>(mm) * n_frames + t] : 0.f;
  }
  float g = -INFINITY;
  for (int i = tid; i < n_blocks; i += 256) g = fmaxf(g, block_max[i]);
  g = group_max<kWave>(g);
  if ((tid & 63) == 0) red[tid >> 6] = g;
  __syncthreads();
  const float floor_v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])) - 8.0f;
#pragma unroll
  for (int q = 0; q < kFinPer; ++q) {
    const int i = tid + 256 * q, mm = i / kTileT, tt = i % kTileT, t = t0 + tt;
    if (t < n_frames) {
      const float r = (fmaxf(v[q], floor_v) + 4.0f) / 4.0f;
      out[static_cast<size_t>(mm) * n_frames + t] = r;
      tile[tt][mm] = f2h(r);
    }
  }
  if (!out16) return;
  __syncthreads();
  for (int i = tid; i < kMels * kTileT; i += 256) {
    const int tt = i / kMels, mm = i % kMels;
    const int t = t0 + tt;
    if (t < n_frames) out16[static_cast<size_t>(t) * kMels + mm] = tile[tt][mm];
  }
}

}  // namespace
}  // namespace fw

extern "C" int64_t fw_log_mel_ws_floats(int n_samples) {
  if (n_samples < fw::kNfft) return 0;
  const int n_frames = n_samples / fw::kHop;
  const int blocks = (n_frames + fw::kFramesPerBlock - 1) / fw::kFramesPerBlock;
  return fw::kWsMax + blocks;
}

extern "C" int fw_log_mel_prepare(const float* filters, float* ws, int64_t ws_floats, hipStream_t stream) {
  if (!filters || !ws) return fw_fail(FW_EINVAL, "log_mel_prepare: null pointer");
  if (ws_floats < fw::kWsMax) return fw_fail(FW_EINVAL, "log_mel_prepare: workspace needs %d floats", fw::kWsMax);
  if (reinterpret_cast<uintptr_t>(ws) & 15u) return fw_fail(FW_EINVAL, "log_mel_prepare: ws must be 16-byte aligned");
  hipLaunchKernelGGL(fw::logmel_prepare_kernel, dim3(1), dim3(1024), 0, stream, filters, ws);
  return fw_check_launch("log_mel prepare");
}

extern "C" int fw_log_mel_run(const float* wave, int n_samples, const float* filters, float* out, void* out16,
                              float* ws, int64_t ws_floats, hipStream_t stream) {
  if (!wave || !filters || !out || !ws) return fw_fail(FW_EINVAL, "log_mel: null pointer");
  if (n_samples < fw::kNfft) return fw_fail(FW_EINVAL, "log_mel: need at least %d samples", fw::kNfft);
  const int n_frames = n_samples / fw::kHop;
  const int blocks = (n_frames + fw::kFramesPerBlock - 1) / fw::kFramesPerBlock;
  const int64_t need = fw_log_mel_ws_floats(n_samples);
  if (ws_floats < need) return fw_fail(FW_EINVAL, "log_mel: workspace needs %lld floats", static_cast<long long>(need));
  if (reinterpret_cast<uintptr_t>(ws) & 15u) return fw_fail(FW_EINVAL, "log_mel: ws must be 16-byte aligned");
  float* maxima = ws + fw::kWsMax;
  hipLaunchKernelGGL(fw::logmel_frames_kernel, dim3(blocks), dim3(256), 0, stream, wave, n_samples, n_frames, filters,
                     ws, out, maxima);
  int rc = fw_check_launch("log_mel frames");
  if (rc != FW_OK) return rc;
  const int tiles = (n_frames + fw::kTileT - 1) / fw::kTileT;
  hipLaunchKernelGGL(fw::logmel_finalize_kernel, dim3(tiles), dim3(256), 0, stream, out,
                     static_cast<_Float16*>(out16), n_frames, maxima, blocks);
  return fw_check_launch("log_mel finalize");
}

// The waveform's trip to the device (custom/model.py:103-104 pads it with zeros on the device and
// copies the samples from pageable memory): the samples are staged into pinned host memory one chunk
// at a time and each chunk's host -> device copy is queued as soon as it is staged, so the DMA of
// chunk i runs while the host stages chunk i + 1; the padding is cleared on the device.
extern "C" int fw_wave_upload(const float* audio, int64_t n, float* staging, float* dev, int64_t n_total,
                              int64_t chunk, hipStream_t stream) {
  if (!audio || !staging || !dev) return fw_fail(FW_EINVAL, "wave_upload: null pointer");
  if (n < 1 || n > n_total || chunk < 1) return fw_fail(FW_EINVAL, "wave_upload: need 0 < n <= n_total and chunk > 0");
  for (int64_t i = 0; i < n; i += chunk) {
    const int64_t m = std::min(chunk, n - i);
    std::memcpy(staging + i, audio + i, static_cast<size_t>(m) * sizeof(float));
    if (hipMemcpyAsync(dev + i, staging + i, static_cast<size_t>(m) * sizeof(float), hipMemcpyHostToDevice, stream) !=
        hipSuccess)
      return fw_fail(FW_EHIP, "wave_upload: hipMemcpyAsync failed");
  }
  if (n < n_total &&
      hipMemsetAsync(dev + n, 0, static_cast<size_t>(n_total - n) * sizeof(float), stream) != hipSuccess)
    return fw_fail(FW_EHIP, "wave_upload: hipMemsetAsync failed");
  return FW_OK;
}

extern "C" int fw_log_mel(const float* wave, int n_samples, const float* filters, float* out, void* out16, float* ws,
                          int64_t ws_floats, hipStream_t stream) {
  if (!wave || !filters || !out || !ws) return fw_fail(FW_EINVAL, "log_mel: null pointer");
  if (n_samples < fw::kNfft) return fw_fail(FW_EINVAL, "log_mel: need at least %d samples", fw::kNfft);
  const int rc = fw_log_mel_prepare(filters, ws, ws_floats, stream);
  if (rc != FW_OK) return rc;
  return fw_log_mel_run(wave, n_samples, filters, out, out16, ws, ws_floats, stream);
}
