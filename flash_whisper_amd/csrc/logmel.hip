// Log-mel front end for gfx950 (replaces the torch.stft path of custom/model.py:93-98, whose
// arithmetic is WhisperFeatureExtractor._torch_extract_fbank_features):
//   frames: centred STFT, n_fft = 400, hop = 160, periodic Hann, reflect padding, last frame dropped
//   power:  |X[k]|^2 for the 201 one-sided bins
//   mel:    filters^T (128 x 201) @ power, log10(max(., 1e-10))
//   final:  max(x, global_max - 8), (x + 4) / 4
// Pass 1 (one block per 16 frames) stages the reflect-padded samples in LDS, applies the window,
// runs a direct 400-point DFT in fp32 against a twiddle table built in fp64, squares, applies the
// filterbank and log10, and writes one block maximum. Pass 2 reduces the block maxima, clamps,
// rescales, and writes the fp16 time-major copy the encoder's conv stem reads.
#include "fw_common.h"

namespace fw {
namespace {

constexpr int kNfft = 400, kHop = 160, kBins = 201, kMels = 128;
constexpr int kFramesPerBlock = 16;
constexpr int kSpan = (kFramesPerBlock - 1) * kHop + kNfft;  // 2800 samples per block

// torch.stft reflect padding (valid for |overhang| < n). Samples staged for frames past the last one
// can overhang further; they are never used, so the index is only clamped into the buffer.
__device__ __forceinline__ int reflect(int i, int n) {
  if (i < 0) i = -i;
  if (i >= n) i = 2 * (n - 1) - i;
  return i < 0 ? 0 : (i >= n ? n - 1 : i);
}

__global__ void __launch_bounds__(256) logmel_frames_kernel(const float* __restrict__ wave, int n_samples,
                                                            int n_frames, const float* __restrict__ filters,
                                                            float* __restrict__ out, float* __restrict__ block_max) {
  __shared__ float xs[kSpan];
  __shared__ __align__(16) float xw[kNfft][kFramesPerBlock];
  __shared__ float2 tw[kNfft];
  __shared__ __align__(16) float pw[kBins][kFramesPerBlock];
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int f0 = blockIdx.x * kFramesPerBlock;
  const int s0 = f0 * kHop - kNfft / 2;

  for (int i = tid; i < kSpan; i += 256) xs[i] = wave[reflect(s0 + i, n_samples)];
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

  const int m = tid & (kMels - 1), fh = tid >> 7;  // 2 groups of 8 frames
  float acc[8];
#pragma unroll
  for (int f = 0; f < 8; ++f) acc[f] = 0.f;
  for (int k = 0; k < kBins; ++k) {
    const float fk = filters[k * kMels + m];
    if (fk != 0.f) {
      const float4* p = reinterpret_cast<const float4*>(&pw[k][fh * 8]);
      const float4 a = p[0], b = p[1];
      acc[0] = fmaf(fk, a.x, acc[0]);
      acc[1] = fmaf(fk, a.y, acc[1]);
      acc[2] = fmaf(fk, a.z, acc[2]);
      acc[3] = fmaf(fk, a.w, acc[3]);
      acc[4] = fmaf(fk, b.x, acc[4]);
      acc[5] = fmaf(fk, b.y, acc[5]);
      acc[6] = fmaf(fk, b.z, acc[6]);
      acc[7] = fmaf(fk, b.w, acc[7]);
    }
  }
  float vmax = -INFINITY;
#pragma unroll
  for (int f = 0; f < 8; ++f) {
    const int t = f0 + fh * 8 + f;
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
  const int n_frames = n_samples / fw::kHop;
  return (n_frames + fw::kFramesPerBlock - 1) / fw::kFramesPerBlock;
}

extern "C" int fw_log_mel(const float* wave, int n_samples, const float* filters, float* out, void* out16, float* ws,
                          int64_t ws_floats, hipStream_t stream) {
  if (!wave || !filters || !out || !ws) return fw_fail(FW_EINVAL, "log_mel: null pointer");
  if (n_samples < fw::kNfft) return fw_fail(FW_EINVAL, "log_mel: need at least %d samples", fw::kNfft);
  const int n_frames = n_samples / fw::kHop;
  const int blocks = static_cast<int>(fw_log_mel_ws_floats(n_samples));
  if (ws_floats < blocks) return fw_fail(FW_EINVAL, "log_mel: workspace needs %d floats", blocks);
  hipLaunchKernelGGL(fw::logmel_frames_kernel, dim3(blocks), dim3(256), 0, stream, wave, n_samples, n_frames, filters,
                     out, ws);
  int rc = fw_check_launch("log_mel frames");
  if (rc != FW_OK) return rc;
  const int tiles = (n_frames + fw::kTileT - 1) / fw::kTileT;
  hipLaunchKernelGGL(fw::logmel_finalize_kernel, dim3(tiles), dim3(256), 0, stream, out,
                     static_cast<_Float16*>(out16), n_frames, ws, blocks);
  return fw_check_launch("log_mel finalize");
}
