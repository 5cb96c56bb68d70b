// Log-mel front end for gfx950 (replaces the torch.stft path of custom/model.py:93-98, whose
// arithmetic is WhisperFeatureExtractor._torch_extract_fbank_features):
//   frames: centred STFT, n_fft = 400, hop = 160, periodic Hann, reflect padding, last frame dropped
//   power:  |X[k]|^2 for the 201 one-sided bins
//   mel:    filters^T (128 x 201) @ power, log10(max(., 1e-10))
//   final:  max(x, global_max - 8), (x + 4) / 4
// Pass 0 (one block) compacts the filterbank: each mel's triangle is a short run of bins, so it keeps
// the first bin, the run length and the run's weights. Pass 1 (one block per 8 frames) stages the
// reflect-padded samples in LDS, applies the window, runs a direct 400-point DFT in fp32 against a
// twiddle table built in fp64, squares, applies the compacted filterbank (the same terms in the same
// order as the dense product, whose other terms are zero) and log10, and writes one block maximum.
// Pass 2 reduces the block maxima, clamps, rescales, and writes the fp16 time-major copy the encoder's
// conv stem reads.
#include "fw_common.h"

namespace fw {
namespace {

constexpr int kNfft = 400, kHop = 160, kBins = 201, kMels = 128;
constexpr int kFramesPerBlock = 8;
constexpr int kSpan = (kFramesPerBlock - 1) * kHop + kNfft;  // 1520 samples per block
constexpr int kRun = 16;  // longest compacted filter run; longer ones are read from the dense filters

// Workspace layout (floats): [0, blocks) block maxima, then per mel {first bin, run length} as ints,
// then per mel kRun weights.
__host__ __device__ constexpr int64_t ws_meta_offset(int blocks) { return (blocks + 3) / 4 * 4; }

__global__ void __launch_bounds__(kMels) logmel_compact_kernel(const float* __restrict__ filters,
                                                               float* __restrict__ ws_meta) {
  const int m = threadIdx.x;
  int lo = -1, hi = -1;
  for (int k = 0; k < kBins; ++k) {
    if (filters[k * kMels + m] != 0.f) {
      if (lo < 0) lo = k;
      hi = k;
    }
  }
  int* range = reinterpret_cast<int*>(ws_meta);
  float* w = ws_meta + 2 * kMels;
  const int len = lo < 0 ? 0 : hi - lo + 1;
  range[2 * m] = lo < 0 ? 0 : lo;
  range[2 * m + 1] = len;
  for (int j = 0; j < kRun; ++j) w[m * kRun + j] = (j < len && len <= kRun) ? filters[(lo + j) * kMels + m] : 0.f;
}

// torch.stft reflect padding (valid for |overhang| < n). Samples staged for frames past the last one
// can overhang further; they are never used, so the index is only clamped into the buffer.
__device__ __forceinline__ int reflect(int i, int n) {
  if (i < 0) i = -i;
  if (i >= n) i = 2 * (n - 1) - i;
  return i < 0 ? 0 : (i >= n ? n - 1 : i);
}

__global__ void __launch_bounds__(256) logmel_frames_kernel(const float* __restrict__ wave, int n_samples,
                                                            int n_frames, const float* __restrict__ filters,
                                                            const float* __restrict__ ws_meta,
                                                            float* __restrict__ out, float* __restrict__ block_max) {
  __shared__ float xs[kSpan];
  __shared__ __align__(16) float xw[kNfft][kFramesPerBlock];
  __shared__ float2 tw[kNfft];
  __shared__ __align__(16) float pw[kBins][kFramesPerBlock];
  __shared__ int2 mrange[kMels];
  __shared__ float mw[kMels * kRun];
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int f0 = blockIdx.x * kFramesPerBlock;
  const int s0 = f0 * kHop - kNfft / 2;

  for (int i = tid; i < kSpan; i += 256) xs[i] = wave[reflect(s0 + i, n_samples)];
  if (tid < kMels) mrange[tid] = reinterpret_cast<const int2*>(ws_meta)[tid];
  for (int i = tid; i < kMels * kRun; i += 256) mw[i] = ws_meta[2 * kMels + i];
  for (int i = tid; i < kNfft; i += 256) {
    double s, c;
    sincospi(static_cast<double>(i) / 200.0, &s, &c);
    tw[i] = make_float2(static_cast<float>(c), static_cast<float>(s));
  }
  __syncthreads();
  for (int i = tid; i < kNfft * kFramesPerBlock; i += 256) {
    const int n = i / kFramesPerBlock, f = i % kFramesPerBlock;
    const float win = 0.5f - 0.5f * tw[n].x;  // periodic Hann: 0.5 - 0.5 cos(2 pi n / 400)
    xw[n][f] = xs[f * kHop + n] * win;
  }
  __syncthreads();

  if (tid < kBins) {
    const int k = tid;
    float re[kFramesPerBlock], im[kFramesPerBlock];
#pragma unroll
    for (int f = 0; f < kFramesPerBlock; ++f) re[f] = im[f] = 0.f;
    int idx = 0;
    for (int n = 0; n < kNfft; ++n) {
      const float2 t = tw[idx];
      const float4* xr = reinterpret_cast<const float4*>(&xw[n][0]);
#pragma unroll
      for (int q = 0; q < kFramesPerBlock / 4; ++q) {
        const float4 x = xr[q];
        re[4 * q + 0] = fmaf(x.x, t.x, re[4 * q + 0]);
        re[4 * q + 1] = fmaf(x.y, t.x, re[4 * q + 1]);
        re[4 * q + 2] = fmaf(x.z, t.x, re[4 * q + 2]);
        re[4 * q + 3] = fmaf(x.w, t.x, re[4 * q + 3]);
        im[4 * q + 0] = fmaf(x.x, t.y, im[4 * q + 0]);
        im[4 * q + 1] = fmaf(x.y, t.y, im[4 * q + 1]);
        im[4 * q + 2] = fmaf(x.z, t.y, im[4 * q + 2]);
        im[4 * q + 3] = fmaf(x.w, t.y, im[4 * q + 3]);
      }
      idx += k;
      if (idx >= kNfft) idx -= kNfft;
    }
#pragma unroll
    for (int f = 0; f < kFramesPerBlock; ++f) pw[k][f] = re[f] * re[f] + im[f] * im[f];
  }
  __syncthreads();

  // filterbank: the nonzero terms of filters^T @ power in increasing bin order, as the dense sum
  const int m = tid & (kMels - 1), fh = tid >> 7;  // 2 groups of 4 frames
  constexpr int kF = kFramesPerBlock / 2;
  float acc[kF];
#pragma unroll
  for (int f = 0; f < kF; ++f) acc[f] = 0.f;
  const int2 rg = mrange[m];
  for (int j = 0; j < rg.y; ++j) {
    const int k = rg.x + j;
    const float fk = rg.y <= kRun ? mw[m * kRun + j] : filters[k * kMels + m];
    if (fk != 0.f) {
      const float4 a = *reinterpret_cast<const float4*>(&pw[k][fh * kF]);
      acc[0] = fmaf(fk, a.x, acc[0]);
      acc[1] = fmaf(fk, a.y, acc[1]);
      acc[2] = fmaf(fk, a.z, acc[2]);
      acc[3] = fmaf(fk, a.w, acc[3]);
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

constexpr int kTileT = 64;

__global__ void __launch_bounds__(256) logmel_finalize_kernel(float* __restrict__ out, _Float16* __restrict__ out16,
                                                              int n_frames, const float* __restrict__ block_max,
                                                              int n_blocks) {
  __shared__ float red[4];
  __shared__ _Float16 tile[kTileT][kMels + 2];
  const int tid = threadIdx.x;
  float g = -INFINITY;
  for (int i = tid; i < n_blocks; i += 256) g = fmaxf(g, block_max[i]);
  g = group_max<kWave>(g);
  if ((tid & 63) == 0) red[tid >> 6] = g;
  __syncthreads();
  const float floor_v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])) - 8.0f;
  const int t0 = blockIdx.x * kTileT;
  for (int i = tid; i < kMels * kTileT; i += 256) {
    const int mm = i / kTileT, tt = i % kTileT;
    const int t = t0 + tt;
    if (t < n_frames) {
      float* p = out + static_cast<size_t>(mm) * n_frames + t;
      const float v = (fmaxf(*p, floor_v) + 4.0f) / 4.0f;
      *p = v;
      tile[tt][mm] = f2h(v);
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
  return fw::ws_meta_offset(blocks) + 2 * fw::kMels + fw::kMels * fw::kRun;
}

extern "C" int fw_log_mel(const float* wave, int n_samples, const float* filters, float* out, void* out16, float* ws,
                          int64_t ws_floats, hipStream_t stream) {
  if (!wave || !filters || !out || !ws) return fw_fail(FW_EINVAL, "log_mel: null pointer");
  if (n_samples < fw::kNfft) return fw_fail(FW_EINVAL, "log_mel: need at least %d samples", fw::kNfft);
  const int n_frames = n_samples / fw::kHop;
  const int blocks = (n_frames + fw::kFramesPerBlock - 1) / fw::kFramesPerBlock;
  const int64_t need = fw_log_mel_ws_floats(n_samples);
  if (ws_floats < need) return fw_fail(FW_EINVAL, "log_mel: workspace needs %lld floats", static_cast<long long>(need));
  if (reinterpret_cast<uintptr_t>(ws) & 15u) return fw_fail(FW_EINVAL, "log_mel: ws must be 16-byte aligned");
  float* meta = ws + fw::ws_meta_offset(blocks);
  hipLaunchKernelGGL(fw::logmel_compact_kernel, dim3(1), dim3(fw::kMels), 0, stream, filters, meta);
  int rc = fw_check_launch("log_mel compact");
  if (rc != FW_OK) return rc;
  hipLaunchKernelGGL(fw::logmel_frames_kernel, dim3(blocks), dim3(256), 0, stream, wave, n_samples, n_frames, filters,
                     meta, out, ws);
  rc = fw_check_launch("log_mel frames");
  if (rc != FW_OK) return rc;
  const int tiles = (n_frames + fw::kTileT - 1) / fw::kTileT;
  hipLaunchKernelGGL(fw::logmel_finalize_kernel, dim3(tiles), dim3(256), 0, stream, out,
                     static_cast<_Float16*>(out16), n_frames, ws, blocks);
  return fw_check_launch("log_mel finalize");
}
