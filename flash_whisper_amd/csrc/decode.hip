// Batch-1 Whisper decoder kernels for gfx950 (wave64). Every launch goes on the caller's stream and
// allocates nothing, so a whole decoder step can be captured into one hipGraph.
//
// Rounding points follow sp4s-s/flash_whisper custom/kernels/whisper_kernels.cu and the fp16
// F.linear chain of custom/model.py:107-123: fp16 residual after every add, fp16 LayerNorm output,
// fp16 GEMV outputs (bias added in fp32 before the single rounding), fp32 softmax with the scale
// applied after the dot, fp16 attention output, fp16-rounded logits before the argmax.
#include <atomic>
#include <mutex>

#include "decode_dev.h"
#include "fw_common.h"

namespace fw {
namespace {

// ------------------------------------------------------------------------------------------
// add_layernorm (reference semantics: h updated in place, y written to global memory).
// ------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) add_layernorm_kernel(_Float16* h, const _Float16* x, const _Float16* gamma,
                                                            const _Float16* beta, _Float16* y, float eps) {
  __shared__ float red[4];
  // Single block: each thread reads its own elements before writing them back, so in-place is safe.
  ln_prologue<256>(h, x, x ? h : nullptr, gamma, beta, eps, y, red);
}

// The final LayerNorm of the LM-head kernels on its own (their 1024-thread reduction order).
__global__ void __launch_bounds__(1024) final_layernorm_kernel(const _Float16* h, const _Float16* x,
                                                               const _Float16* gamma, const _Float16* beta,
                                                               _Float16* y, float eps) {
  __shared__ float red[2 * 1024 / kWave];
  LnRegs<1024> in;
  ln_load<1024>(h, x, gamma, beta, in);
  ln_finish<1024, true>(in, x != nullptr, nullptr, eps, y, red);
}

__global__ void __launch_bounds__(256) embed_kernel(const int64_t* cur, const int64_t* state, const _Float16* embed,
                                                    const _Float16* pos_embed, int vocab, int max_pos, _Float16* h) {
  const _Float16 *a, *b;
  embed_rows(cur, state, embed, pos_embed, vocab, max_pos, &a, &b);
  for (int i = threadIdx.x; i < kHidden; i += blockDim.x) h[i] = f2h(h2f(a[i]) + h2f(b[i]));
}

// ------------------------------------------------------------------------------------------
// GEMV: out[n] = act(fp16(W[n,:] . x + bias[n])). Each row is split over kLPR lanes that stream
// 16-byte chunks; a wave covers 64 / kLPR rows at once and U row groups are loaded before any
// arithmetic so every lane keeps U * kC 16-byte loads in flight. Blocks own contiguous row ranges.
// With LN, the 1280-wide input is the LayerNorm of the residual, computed per block into LDS.
// ------------------------------------------------------------------------------------------

// NV input vectors (a batch of decoder positions, NV <= kMaxBatch) share every weight row load: vector
// v reads x / h / h_out at offset v * K and writes out + v * n; its LN or combine prologue is that of
// a single-vector launch, so each vector's result is bit-identical to NV separate launches.
template <int K, int NW, int U, int MODE, int ACT, int NV = 1>
__global__ void __launch_bounds__(NW * 64) gemv_kernel(const _Float16* __restrict__ xin, LnArgs ln, CombineArgs cb,
                                                       const _Float16* __restrict__ w,
                                                       const _Float16* __restrict__ bias, _Float16* __restrict__ out,
                                                       int n) {
  using RS = RowSplit<K>;
  constexpr int kRowsPerBlock = NW * RS::kRPW * U;
  __shared__ __align__(16) _Float16 y_lds[MODE != kModePlain ? NV * K : 8];
  __shared__ float red[MODE == kModeLn ? 2 * NV * NW : NW];
  __shared__ float wgt[MODE == kModeCombine ? kMaxCombineHeads * kMaxCombineSplits : 1];
  __shared__ float inv_den[MODE == kModeCombine ? kMaxCombineHeads : 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % RS::kLPR, rsel = lane / RS::kLPR;
  // Order of requests: the prologue's inputs (small, on the critical path), then this block's weight
  // rows, which do not depend on the input vector and stay in flight while the prologue computes.
  LnRegs<NW * 64> lnr[MODE == kModeLn ? NV : 1];
  // one vector at a time; a batch keeps the next vector's partials in flight while one is merged
  CombineRegs<MODE == kModeCombine ? NW * 64 : 64> cbr[MODE == kModeCombine && NV > 1 ? 2 : 1];
  if constexpr (MODE == kModeLn) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const _Float16* a = ln.h ? ln.h + v * kHidden : nullptr;
      const _Float16* b = ln.x ? ln.x + v * kHidden : nullptr;
      if (ln.cur) embed_rows(ln.cur, ln.state, ln.embed, ln.pos_embed, ln.vocab, ln.max_pos, &a, &b, v);
      ln_load<NW * 64>(a, b, ln.gamma, ln.beta, lnr[v]);
    }
  } else if constexpr (MODE == kModeCombine) {
    combine_load<NW * 64>(NV > 1 ? cb.vec(0) : cb, cbr[0]);
  }
  const int row0 = blockIdx.x * kRowsPerBlock + wave * RS::kRPW * U + rsel;
  // Rows past n load row n - 1 (their results are never stored): no load sits under a lane mask,
  // so none of them forces a wait for the loads before it. The bias is requested first, so waiting
  // for it never waits for a weight row.
  _Float16 braw[U];
#pragma unroll
  for (int u = 0; u < U; ++u) braw[u] = *(bias ? bias + min(row0 + u * RS::kRPW, n - 1) : &g_zero_half);
  const uint4* w4 = reinterpret_cast<const uint4*>(w);
  uint4 wr[U][RS::kC];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const size_t row = min(row0 + u * RS::kRPW, n - 1);
#pragma unroll
    for (int c = 0; c < RS::kC; ++c) wr[u][c] = ld_weights(w4 + row * RS::kChunksRow + sub + RS::kLPR * c);
  }
  const uint4* xv;
  if constexpr (MODE == kModeLn) {
    if constexpr (NV == 1)
      ln_finish<NW * 64, true>(lnr[0], ln.cur != nullptr || ln.x != nullptr, ln.h_out, ln.eps, y_lds, red);
    else
      ln_finish_multi<NW * 64, NV>(lnr, ln.cur != nullptr || ln.x != nullptr, ln.h_out, ln.eps, y_lds, red);
    __syncthreads();
    xv = reinterpret_cast<const uint4*>(y_lds);
  } else if constexpr (MODE == kModeCombine) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      if (v + 1 < NV) combine_load<NW * 64>(cb.vec(v + 1), cbr[(v + 1) & 1]);
      combine_finish<NW * 64>(NV > 1 ? cb.vec(v) : cb, cbr[v & 1], y_lds + v * K, wgt, inv_den);
      __syncthreads();  // y visible; wgt / inv_den free for the next vector
    }
    xv = reinterpret_cast<const uint4*>(y_lds);
  } else {
    xv = reinterpret_cast<const uint4*>(xin);
  }
  uint4 xr[NV][RS::kC];
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int c = 0; c < RS::kC; ++c) xr[v][c] = xv[v * (K / 8) + sub + RS::kLPR * c];

#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int row = row0 + u * RS::kRPW;
    const float b = h2f(braw[u]);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      float acc = 0.f;
#pragma unroll
      for (int c = 0; c < RS::kC; ++c) acc = dot8(wr[u][c], xr[v][c], acc);
      acc = group_sum<RS::kLPR>(acc);
      // every lane finishes the row and one lane stores; the empty asm pins y (and with it the
      // bias) outside the store's lane mask, where the bias request would otherwise be sunk to
      float y = acc + b;
      if constexpr (ACT == FW_ACT_GELU) y = gelu_erf(round_h(y));
      asm volatile("" : "+v"(y));
      if (sub == 0 && row < n) out[static_cast<size_t>(v) * n + row] = f2h(y);
    }
  }
}

constexpr int kMaxBatch = 4;  // decoder positions per batched launch (the 4-token prompt)

template <int K, int NW, int U, int MODE, int ACT, int NV = 1>
void launch_gemv(const _Float16* x, const LnArgs& ln, const CombineArgs& cb, const _Float16* w, const _Float16* b,
                 _Float16* out, int n, hipStream_t s) {
  constexpr int kRows = NW * RowSplit<K>::kRPW * U;
  const int grid = (n + kRows - 1) / kRows;
  hipLaunchKernelGGL((gemv_kernel<K, NW, U, MODE, ACT, NV>), dim3(grid), dim3(NW * 64), 0, s, x, ln, cb, w, b, out, n);
}

// A batch of nv (1..kMaxBatch) vectors, one row group per wave (the batch runs once per clip, for the
// prompt, so registers for up to 4 input vectors matter more than the row-group depth). NW is that of
// the single-vector launch of the same weights: the LayerNorm prologue reduces over the block's
// threads, and the same block size keeps each vector's result bit-identical to a single-vector step.
template <int K, int NW, int MODE, int ACT>
void launch_gemv_batch(int nv, const _Float16* x, const LnArgs& ln, const CombineArgs& cb, const _Float16* w,
                       const _Float16* b, _Float16* out, int n, hipStream_t s) {
  switch (nv) {
    case 1: launch_gemv<K, NW, 1, MODE, ACT, 1>(x, ln, cb, w, b, out, n, s); break;
    case 2: launch_gemv<K, NW, 1, MODE, ACT, 2>(x, ln, cb, w, b, out, n, s); break;
    case 3: launch_gemv<K, NW, 1, MODE, ACT, 3>(x, ln, cb, w, b, out, n, s); break;
    default: launch_gemv<K, NW, 1, MODE, ACT, 4>(x, ln, cb, w, b, out, n, s); break;
  }
}

// Block shapes of the decode GEMVs (waves per block, row groups per wave), measured on MI355X over the
// whole decoder step (alternating runs of each shape on one device): large blocks (8-12 waves, 54-160
// blocks) beat one small block per CU because the prologue (LayerNorm or split-K combine) is repeated
// per block and its latency is the critical path; 4- and 16-wave blocks were slower everywhere.
#ifndef FW_G5120_NW
#define FW_G5120_NW 8  // LN + fc1 (5120 rows): 32 rows per block
#endif
#ifndef FW_G5120_U
#define FW_G5120_U 2
#endif
#ifndef FW_G3840_NW
#define FW_G3840_NW 8  // LN + q/k/v (3840 rows): 16 rows per block
#endif
#ifndef FW_G3840_U
#define FW_G3840_U 1
#endif
#ifndef FW_G1280_NW
#define FW_G1280_NW 8  // LN + cross q (1280 rows): 16 rows per block
#endif
#ifndef FW_GK5120_NW
#define FW_GK5120_NW 8  // fc2 (K = 5120): 8 rows per block
#endif
#ifndef FW_GK5120_U
#define FW_GK5120_U 1
#endif
#ifndef FW_CMB_NW
#define FW_CMB_NW 12  // combine + out projection: 24 rows per block
#endif
// Block shapes are whole blocks within the 1024-thread launch bound with at least one row group per
// wave; any such shape computes the same rows (each row's lane split and order depend on K only).
// The LayerNorm prologue of a shape fixes its reduction order, so the batched prompt launches reuse
// the single-vector block sizes.
#define FW_GEMV_SHAPE_OK(NW, U) ((NW) >= 1 && (NW) <= 16 && (U) >= 1 && (U) <= 4)
static_assert(FW_GEMV_SHAPE_OK(FW_G5120_NW, FW_G5120_U) && FW_GEMV_SHAPE_OK(FW_G3840_NW, FW_G3840_U) &&
                  FW_GEMV_SHAPE_OK(FW_G1280_NW, 1) && FW_GEMV_SHAPE_OK(FW_GK5120_NW, FW_GK5120_U) &&
                  FW_GEMV_SHAPE_OK(FW_CMB_NW, 1),
              "decode GEMV block shapes: 1..16 waves, 1..4 row groups per wave");
#undef FW_GEMV_SHAPE_OK
template <int MODE, int ACT>
void dispatch_gemv_1280(const _Float16* x, const LnArgs& ln, const CombineArgs& cb, const _Float16* w,
                        const _Float16* b, _Float16* out, int n, hipStream_t s) {
  if (n >= 5120)
    launch_gemv<kHidden, FW_G5120_NW, FW_G5120_U, MODE, ACT>(x, ln, cb, w, b, out, n, s);
  else if (n >= 3840)
    launch_gemv<kHidden, FW_G3840_NW, FW_G3840_U, MODE, ACT>(x, ln, cb, w, b, out, n, s);
  else
    launch_gemv<kHidden, FW_G1280_NW, 1, MODE, ACT>(x, ln, cb, w, b, out, n, s);
}

template <int MODE, int ACT>
void dispatch_gemv_1280_batch(int nv, const _Float16* x, const LnArgs& ln, const CombineArgs& cb, const _Float16* w,
                              const _Float16* b, _Float16* out, int n, hipStream_t s) {
  if (nv == 1)
    dispatch_gemv_1280<MODE, ACT>(x, ln, cb, w, b, out, n, s);
  else if (n >= 5120)
    launch_gemv_batch<kHidden, FW_G5120_NW, MODE, ACT>(nv, x, ln, cb, w, b, out, n, s);
  else if (n >= 3840)
    launch_gemv_batch<kHidden, FW_G3840_NW, MODE, ACT>(nv, x, ln, cb, w, b, out, n, s);
  else
    launch_gemv_batch<kHidden, FW_G1280_NW, MODE, ACT>(nv, x, ln, cb, w, b, out, n, s);
}

// ------------------------------------------------------------------------------------------
// LM head + argmax (reference lm_head_argmax_kernel, whisper_kernels.cu:28-86): rows of the tied
// embedding are streamed once; each row's fp32 dot is rounded to fp16, packed with its index and
// max-reduced to one 64-bit atomicMax per block. The logits vector is never written. Blocks take
// 64-row batches round-robin; a block's first batch is requested before the (optional)
// final-LayerNorm prologue and the next batch is always in flight while one is scored (two register
// buffers per wave). The finalize step (reference argmax_finalize_kernel, :88-100) is a separate
// 1-thread launch: a last-block-done finalize needs a device-scope release per block, which on this
// part writes back the L2 and costs more than the extra launch (measured +2.8 us per decode step).
// ------------------------------------------------------------------------------------------
#ifndef FW_LM_NW
#define FW_LM_NW 16
#endif
#ifndef FW_LM_U
#define FW_LM_U 2
#endif
// The int8 pre-pass kernel scores one row per 16 lanes (64 rows a batch at 16 waves, so two row groups
// per wave in the fp16 kernel's layout) and gives each pair of the 1280 y values its own thread.
static_assert(FW_LM_U == 2, "FW_LM_U: the int8 LM head shares the fp16 head's batch of 4 rows per wave");
static_assert(FW_LM_NW >= 10 && FW_LM_NW <= 16, "FW_LM_NW: 640..1024 threads (one per pair of y values)");
#ifndef FW_LM_BPC
#define FW_LM_BPC 1  // fp16 LM head: blocks per CU the grid is sized for
#endif
static_assert(FW_LM_BPC >= 1 && FW_LM_BPC <= 4, "FW_LM_BPC: 1..4 blocks per CU");

constexpr int kLmNW = FW_LM_NW, kLmU = FW_LM_U;
constexpr int kLmRowsIter = kLmNW * 2 * kLmU;  // rows per block iteration


template <bool LN>
__global__ void __launch_bounds__(kLmNW * 64) lm_head_kernel(const _Float16* __restrict__ yin, LnArgs ln,
                                                             const _Float16* __restrict__ w,
                                                             const uint8_t* __restrict__ suppress, int vocab,
                                                             unsigned long long* best) {
  using RS = RowSplit<kHidden>;
  __shared__ __align__(16) _Float16 y_lds[kHidden];
  __shared__ float red[kLmNW];
  __shared__ unsigned long long block_best[kLmNW * 2];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane & 31, rsel = lane >> 5;
  const uint4* w4 = reinterpret_cast<const uint4*>(w);
  // Batches of kLmRowsIter rows are dealt to the blocks round-robin: batch k of this block starts at
  // row (k * gridDim.x + blockIdx.x) * kLmRowsIter, so at any moment the grid streams one contiguous
  // stretch of the table.
  const int r_end = vocab;
  auto base_of = [&](int k) { return (k * static_cast<int>(gridDim.x) + static_cast<int>(blockIdx.x)) * kLmRowsIter; };

  // Rows past r_end load row r_end - 1 and are masked when scored: no load sits under a lane mask,
  // so the wait for one batch never includes the batch requested after it.
  auto load = [&](int base, uint4 (&wr)[kLmU][RS::kC], uint32_t (&sp)[kLmU]) {
    const int row0 = base + wave * 2 * kLmU + rsel;
#pragma unroll
    for (int u = 0; u < kLmU; ++u) {
      const size_t row = min(row0 + 2 * u, r_end - 1);
#pragma unroll
      for (int c = 0; c < RS::kC; ++c) wr[u][c] = ld_lm_head(w4 + row * RS::kChunksRow + sub + 32 * c);
      sp[u] = suppress[row];
    }
  };
  LnRegs<kLmNW * 64> lnr;
  if constexpr (LN) ln_load<kLmNW * 64>(ln.h, ln.x, ln.gamma, ln.beta, lnr);
  uint4 wa[kLmU][RS::kC], wb[kLmU][RS::kC];
  uint32_t sa[kLmU], sb[kLmU];
  load(base_of(0), wa, sa);

  if constexpr (LN) {
    ln_finish<kLmNW * 64>(lnr, ln.x != nullptr, nullptr, ln.eps, y_lds, red);
  } else {
    for (int i = threadIdx.x; i < kHidden / 8; i += blockDim.x)
      reinterpret_cast<uint4*>(y_lds)[i] = reinterpret_cast<const uint4*>(yin)[i];
  }
  __syncthreads();
  uint4 xr[RS::kC];
#pragma unroll
  for (int c = 0; c < RS::kC; ++c) xr[c] = reinterpret_cast<const uint4*>(y_lds)[sub + 32 * c];

  unsigned long long mine = 0;
  auto score = [&](int base, const uint4 (&wr)[kLmU][RS::kC], const uint32_t (&sp)[kLmU]) {
    const int row0 = base + wave * 2 * kLmU + rsel;
#pragma unroll
    for (int u = 0; u < kLmU; ++u) {
      const int row = row0 + 2 * u;
      float acc = 0.f;
#pragma unroll
      for (int c = 0; c < RS::kC; ++c) acc = dot8(wr[u][c], xr[c], acc);
      acc = group_sum<32>(acc);  // every lane of the row holds the sum
      const unsigned long long sc = pack_score(round_h(acc), row);
      if (row < r_end && !sp[u] && sc > mine) mine = sc;
    }
  };
  // two register buffers in turn: batch i + 1 is in flight while batch i is scored
  for (int k = 0; base_of(k) < r_end; k += 2) {
    const int base = base_of(k), b1 = base_of(k + 1), b2 = base_of(k + 2);
    if (b1 < r_end) load(b1, wb, sb);
    score(base, wa, sa);
    if (b2 < r_end) load(b2, wa, sa);
    if (b1 < r_end) score(b1, wb, sb);
  }
  if (sub == 0) block_best[wave * 2 + rsel] = mine;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long m = 0;
#pragma unroll
    for (int i = 0; i < kLmNW * 2; ++i) m = block_best[i] > m ? block_best[i] : m;
    if (m) atomicMax(best, m);
  }
}

int lm_head_grid(int vocab) {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess &&
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus = 256;
  // as few batches per block as the CUs allow, then as few blocks as that count needs
  const int batches = (vocab + kLmRowsIter - 1) / kLmRowsIter;
  const int per = (batches + cus * FW_LM_BPC - 1) / (cus * FW_LM_BPC);
  return (batches + per - 1) / per;
}

__global__ void argmax_finalize_kernel(unsigned long long* best, FinArgs fin) { finalize_token(best, fin); }

// ------------------------------------------------------------------------------------------
// LM head with an int8 pre-pass: the packed winner of lm_head_kernel, bit for bit, from about half
// of its HBM bytes. The embedding is also kept as int8 rows q_v with a per-row scale s_v and a per-row
// bound e_v >= || E_v - s_v q_v ||_2 (lm_q8_pack_kernel). Each block, over its 256 rows:
//  1. scores them on the int8 table. y is quantized per block to integers y_int of step t
//     (|y_int| <= 127 * 128), split into two int8 digits, so q_v . y_int is an exact integer dot
//     (v_dot4_i32_i8) and A_v = s_v t (q_v . y_int) takes one fp64 rounding. With eta = y - t y_int,
//     |Ehat_v| <= 127 s_v sqrt(1280) + e_v =: nE_v (a bound on |E_v| and |s_v q_v|) and
//     g = 1280 * 2^-24 / (1 - 1280 * 2^-24), the fp32 logit X_v that lm_head_kernel computes obeys
//       |A_v - X_v| <= r_v = |y| e_v + (|eta| + g |y|) nE_v
//     (quantization of E, quantization of y, and the fp32 rounding of X_v, whose dot has at most 45
//     roundings, each at most 2^-24 of the sum of |products| <= |y| |E_v|); r_v is inflated by 2^-20
//     and the bounds A_v -+ r_v are rounded outward to fp32;
//  2. takes T = max(A_v - r_v) over its unsuppressed rows. Some row has X >= T, so the block's winner w
//     has fp16(X_w) >= fp16(T) and X_w >= T - (two fp16 spacings at T) >= thr(T) (below): every row
//     with A_v + r_v >= thr is a candidate, and every row that ties the winner is one too;
//  3. computes each candidate's logit with exactly the lane split and summation order of
//     lm_head_kernel, packs it as that kernel does and sends the block maximum to best with one
//     atomicMax. The maximum over blocks is then that of lm_head_kernel.
// Candidates are typically 0-15 of a block's 256 rows for fp16 logits of unit scale; when every logit
// is equal (y = 0) all rows are candidates and the block reads its fp16 rows as lm_head_kernel does.
// ------------------------------------------------------------------------------------------
constexpr int kQ8RowsPerBlock = kLmRowsIter * 4;  // 4 batches of 64 rows, dealt round-robin
static_assert(kLmNW * 64 / kQ8Lpr == kLmRowsIter, "one int8 row per 16 lanes per batch");
static_assert(kLmNW * 64 >= kHidden / 2, "the y statistics and digits take one thread per pair of y values");

__global__ void __launch_bounds__(256) lm_q8_pack_kernel(const _Float16* __restrict__ w, int vocab,
                                                         int8_t* __restrict__ wq, float2* __restrict__ meta) {
  constexpr int kPer = kHidden / 64;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= vocab) return;  // wave-uniform
  const _Float16* wr = w + static_cast<size_t>(row) * kHidden;
  float v[kPer];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    v[i] = h2f(wr[lane + 64 * i]);
    amax = fmaxf(amax, fabsf(v[i]));
  }
  amax = group_max<64>(amax);
  const float s = amax / 127.0f;
  const float inv = amax > 0.f ? 127.0f / amax : 0.f;
  double err = 0.0;
  int8_t* qr = wq + static_cast<size_t>(row) * kHidden;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const float q = fminf(fmaxf(rintf(v[i] * inv), -127.f), 127.f);
    qr[lane + 64 * i] = static_cast<int8_t>(q);
    const double d = static_cast<double>(v[i]) - static_cast<double>(s) * static_cast<double>(q);
    err = fma(d, d, err);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) err += __shfl_xor(err, o);
  if (lane == 0) meta[row] = make_float2(s, __double2float_ru(sqrt(err) * (1.0 + 0x1p-40)));
}

template <bool LN>
__global__ void __launch_bounds__(kLmNW * 64) lm_head_q8_kernel(const _Float16* __restrict__ yin, LnArgs ln,
                                                                const _Float16* __restrict__ w,
                                                                const int8_t* __restrict__ wq,
                                                                const float2* __restrict__ meta,
                                                                const uint8_t* __restrict__ suppress, int vocab,
                                                                unsigned long long* best) {
  __shared__ __align__(16) _Float16 y_lds[kHidden];
  __shared__ __align__(16) int8_t yhi[kHidden];
  __shared__ __align__(16) int8_t ylo[kHidden];
  __shared__ float red[4 * kLmNW];  // LayerNorm sums, then max |y| and |y|^2: a slot set per round
  __shared__ float ub_lds[kQ8RowsPerBlock];
  __shared__ int cand[kQ8RowsPerBlock];
  __shared__ int ncand;
  __shared__ unsigned long long block_best[kLmNW * 2];
  constexpr int kNT = kLmNW * 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane & (kQ8Lpr - 1), rsel = lane / kQ8Lpr;  // 4 rows per wave
  const uint4* wq4 = reinterpret_cast<const uint4*>(wq);
  auto base_of = [&](int k) { return (k * static_cast<int>(gridDim.x) + static_cast<int>(blockIdx.x)) * kLmRowsIter; };

  struct Batch {
    uint4 w[kQ8C];
    float2 m;
    uint32_t sp;
  };
  // Rows past vocab load row vocab - 1 (no load under a lane mask) and are dropped when scored.
  auto load = [&](int base, Batch& b) {
    const size_t row = min(base + wave * 4 + rsel, vocab - 1);
#pragma unroll
    for (int c = 0; c < kQ8C; ++c) b.w[c] = ld_lm_head(wq4 + row * kQ8Chunks + sub + kQ8Lpr * c);
    b.m = meta[row];
    b.sp = suppress[row];
  };
  LnRegs<kNT> lnr;
  if constexpr (LN) ln_load<kNT>(ln.h, ln.x, ln.gamma, ln.beta, lnr);
  if (tid == 0) ncand = 0;
  // The first batch is requested before the LayerNorm, the second after it, the other two as soon as a
  // register buffer frees up. About one 82 KB batch per CU in flight streams faster than more: with
  // two requested up front the launch took 0.5 us longer, with all four 3 us longer (the table's DRAM
  // pages are then visited by many more interleaved request streams).
  Batch ba, bb;
  load(base_of(0), ba);

  if constexpr (LN) {
    ln_finish<kNT, true>(lnr, ln.x != nullptr, nullptr, ln.eps, y_lds, red);  // thread tid owns pair tid
  } else {
    for (int i = tid; i < kHidden / 8; i += kNT)
      reinterpret_cast<uint4*>(y_lds)[i] = reinterpret_cast<const uint4*>(yin)[i];
    __syncthreads();
  }
  load(base_of(1), bb);
  // y statistics in one reduction round: max |y| and |y|^2. Then y_int = rint(y / t) in two int8 digits.
  constexpr int kPairs = kHidden / 2;
  const bool has_pair = tid < kPairs;
  h2v yp = {static_cast<_Float16>(0.f), static_cast<_Float16>(0.f)};
  if (has_pair) yp = reinterpret_cast<const h2v*>(y_lds)[tid];
  const float y0 = h2f(yp.x), y1 = h2f(yp.y);
  const float wmax = group_max<64>(fmaxf(fabsf(y0), fabsf(y1)));
  const float wsq = group_sum<64>(y0 * y0 + y1 * y1);
  if (lane == 0) {
    red[2 * kLmNW + wave] = wmax;
    red[3 * kLmNW + wave] = wsq;
  }
  __syncthreads();
  float amax = 0.f, ysq = 0.f;
#pragma unroll
  for (int i = 0; i < kLmNW; ++i) {
    amax = fmaxf(amax, red[2 * kLmNW + i]);
    ysq += red[3 * kLmNW + i];
  }
  const float tinv = amax > 0.f ? static_cast<float>(kQ8YMax) / amax : 0.f;
  if (has_pair) {
    const int n0 = static_cast<int>(fminf(fmaxf(rintf(y0 * tinv), -kQ8YMax), kQ8YMax));
    const int n1 = static_cast<int>(fminf(fmaxf(rintf(y1 * tinv), -kQ8YMax), kQ8YMax));
    const int h0 = (n0 + 64) >> 7, h1 = (n1 + 64) >> 7;  // floor division; lo digits in [-64, 63]
    yhi[2 * tid] = static_cast<int8_t>(h0);
    yhi[2 * tid + 1] = static_cast<int8_t>(h1);
    ylo[2 * tid] = static_cast<int8_t>(n0 - 128 * h0);
    ylo[2 * tid + 1] = static_cast<int8_t>(n1 - 128 * h1);
  }
  __syncthreads();  // publishes the digits and y_lds
  const Q8Step q8 = q8_step(amax, ysq);  // the same t as above
  uint4 dh[kQ8C], dl[kQ8C];
#pragma unroll
  for (int c = 0; c < kQ8C; ++c) {
    dh[c] = reinterpret_cast<const uint4*>(yhi)[sub + kQ8Lpr * c];
    dl[c] = reinterpret_cast<const uint4*>(ylo)[sub + kQ8Lpr * c];
  }

  float lb_max = -INFINITY;
  auto score = [&](int k, const Batch& b) {
    const int slot_row = wave * 4 + rsel;
    const int row = base_of(k) + slot_row;
    int ah = 0, al = 0;
#pragma unroll
    for (int c = 0; c < kQ8C; ++c) {
      ah = dot16_i8(b.w[c], dh[c], ah);
      al = dot16_i8(b.w[c], dl[c], al);
    }
    ah = xor_add_i16(ah);
    al = xor_add_i16(al);
    float ub, lb;
    q8_bounds(ah, al, b.m, q8, ub, lb);
    const bool live = row < vocab && !b.sp;
    ub = live ? ub : -INFINITY;
    lb = live ? lb : -INFINITY;
    lb_max = fmaxf(lb_max, lb);
    if (sub == 0) ub_lds[k * kLmRowsIter + slot_row] = ub;
  };
  // 4 batches, two register buffers in turn
  score(0, ba);
  load(base_of(2), ba);
  score(1, bb);
  load(base_of(3), bb);
  score(2, ba);
  score(3, bb);

  lb_max = group_max<64>(lb_max);
  if (lane == 0) red[wave] = lb_max;
  __syncthreads();  // also publishes ub_lds
  float tb = -INFINITY;
#pragma unroll
  for (int i = 0; i < kLmNW; ++i) tb = fmaxf(tb, red[i]);
  const float thr = q8_threshold(tb);
  if (tid < kQ8RowsPerBlock) {
    const int row = base_of(tid / kLmRowsIter) + tid % kLmRowsIter;
    const float ub = ub_lds[tid];
    if (row < vocab && ub != -INFINITY && !(ub < thr)) cand[atomicAdd(&ncand, 1)] = row;
  }
  __syncthreads();

  // exact logits of the candidates: the lane split and order of lm_head_kernel
  using RS = RowSplit<kHidden>;
  const int sub32 = lane & 31, rsel32 = lane >> 5;
  const uint4* w4 = reinterpret_cast<const uint4*>(w);
  uint4 xr[RS::kC];
#pragma unroll
  for (int c = 0; c < RS::kC; ++c) xr[c] = reinterpret_cast<const uint4*>(y_lds)[sub32 + 32 * c];
  const int nc = ncand;
  unsigned long long mine = 0;
  for (int i0c = wave * 2; i0c < nc; i0c += kLmNW * 2) {
    const int i = i0c + rsel32;
    const int row = cand[i < nc ? i : i0c];
    uint4 wr[RS::kC];
#pragma unroll
    for (int c = 0; c < RS::kC; ++c) wr[c] = ld_lm_head(w4 + static_cast<size_t>(row) * RS::kChunksRow + sub32 + 32 * c);
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < RS::kC; ++c) acc = dot8(wr[c], xr[c], acc);
    acc = group_sum<32>(acc);
    const unsigned long long sc = pack_score(round_h(acc), row);
    if (i < nc && sc > mine) mine = sc;
  }
  if (sub32 == 0) block_best[wave * 2 + rsel32] = mine;
  __syncthreads();
  if (tid == 0) {
    unsigned long long m = 0;
#pragma unroll
    for (int i = 0; i < kLmNW * 2; ++i) m = block_best[i] > m ? block_best[i] : m;
    if (m) atomicMax(best, m);
  }
}

int lm_head_q8_grid(int vocab) {
  const int batches = (vocab + kLmRowsIter - 1) / kLmRowsIter;
  return (batches + 3) / 4;
}


// BATCH: a batch of queries (grid.z, the prompt) takes the fresh K/V rows of the batch's earlier
// queries straight from k_new / v_new: their cache rows are written by other blocks of the same
// launch, so a cache row at or past the batch's first position is never trusted. The single-query
// instantiation carries none of this code.
template <int MAXP, bool BATCH, int NW = 4>
__global__ void __launch_bounds__(NW * 64) attn_split_kernel(AttnArgs a) {
  __shared__ float wm[NW], wl[NW];
  __shared__ float wacc[NW][kHeadDim];
  const int split = blockIdx.x, head = blockIdx.y, nsplit = gridDim.x, qv = BATCH ? blockIdx.z : 0;
  const int slot = (qv * gridDim.y + head) * nsplit + split;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ks = lane >> 3, c = lane & 7;
  const size_t hoff = static_cast<size_t>(head) * a.max_len * kHeadDim;
  _Float16* kh = a.k + hoff;
  _Float16* vh = a.v + hoff;
  const size_t kv_off = BATCH ? static_cast<size_t>(qv) * a.kv_stride : 0;
  const uint4* kn = a.k_new ? reinterpret_cast<const uint4*>(a.k_new + kv_off + head * kHeadDim) : nullptr;
  const uint4* vn = a.v_new ? reinterpret_cast<const uint4*>(a.v_new + kv_off + head * kHeadDim) : nullptr;
  // Every wave owns a fixed run of MAXP * 8 keys of the split. All loads are issued before the
  // cached length is known (it arrives from device memory); keys past it are masked afterwards,
  // so the length read and the K/V reads take one memory round trip together.
  const int begin = split * a.split_keys;
  const int w0 = begin + wave * MAXP * 8;
  const int wend = min(min(w0 + MAXP * 8, begin + a.split_keys), a.max_len);
  const int64_t pos_raw = a.len_state ? a.len_state[0] : 0;
  const size_t q_off = BATCH ? static_cast<size_t>(qv) * a.q_stride : 0;
  const uint4 qc = reinterpret_cast<const uint4*>(a.q + q_off + head * kHeadDim)[c];
  uint4 knew = make_uint4(0, 0, 0, 0), vnew = make_uint4(0, 0, 0, 0);
  if (kn) {
    knew = kn[c];
    vnew = vn[c];
  }
  uint4 kr[MAXP], vr[MAXP];
#pragma unroll
  for (int p = 0; p < MAXP; ++p) {
    // keys past wend load row wend - 1 (no load under a lane mask); split_wave_partial masks them
    const int j = min(w0 + p * 8 + ks, wend - 1);
    kr[p] = reinterpret_cast<const uint4*>(kh + static_cast<size_t>(j) * kHeadDim)[c];
    vr[p] = reinterpret_cast<const uint4*>(vh + static_cast<size_t>(j) * kHeadDim)[c];
  }
  const int pos0 = a.len_state ? static_cast<int>(pos_raw < 0 ? 0 : (pos_raw >= a.max_len ? a.max_len - 1 : pos_raw))
                               : -1;
  const int pos = a.len_state ? (BATCH ? min(pos0 + qv, a.max_len - 1) : pos0) : -1;
  const int len = a.len_state ? pos + 1 : a.max_len;
  const int n = min(a.split_keys, len - begin);
  if (n <= 0) {
    if (tid == 0) {
      a.part_m[slot] = -INFINITY;
      a.part_l[slot] = 0.f;
    }
    return;
  }
  if (kn && pos >= begin && pos < begin + n && tid < 16) {
    if (tid < 8)
      reinterpret_cast<uint4*>(kh + static_cast<size_t>(pos) * kHeadDim)[tid] = knew;
    else
      reinterpret_cast<uint4*>(vh + static_cast<size_t>(pos) * kHeadDim)[tid - 8] = vnew;
  }
  const int w1 = min(wend, begin + n);
#pragma unroll
  for (int p = 0; p < MAXP; ++p) {
    const int j = w0 + p * 8 + ks;
    if (kn && j == pos) {  // the new row replaces the (stale) cached one
      kr[p] = knew;
      vr[p] = vnew;
    } else if (BATCH && kn && j >= pos0 && j < pos) {  // an earlier query of the batch: its fresh row
      const size_t r = static_cast<size_t>(j - pos0) * a.kv_stride + head * kHeadDim;
      kr[p] = reinterpret_cast<const uint4*>(a.k_new + r)[c];
      vr[p] = reinterpret_cast<const uint4*>(a.v_new + r)[c];
    }
  }
  split_wave_partial<MAXP>(kr, vr, qc, w0, w1, a.scale, wm + wave, wl + wave, wacc[wave]);
  __syncthreads();
  split_merge_store<NW>(wm, wl, wacc, a, slot);
}

// Splits of up to 256 keys (the cross attention): FW_ATTN256_P passes of 8 keys per wave, 32 / P waves
// (decode_dev.h; the one-launch step's cross attention has the same layout).
int launch_attn_split(const AttnArgs& a, int nsplit, int heads, hipStream_t s, int nq = 1) {
  const dim3 grid(nsplit, heads, nq);
  constexpr int kP256 = FW_ATTN256_P, kW256 = 32 / FW_ATTN256_P;
  if (nq == 1) {
    if (a.split_keys <= 64)
      hipLaunchKernelGGL((attn_split_kernel<2, false>), grid, dim3(256), 0, s, a);
    else if (a.split_keys <= 128)
      hipLaunchKernelGGL((attn_split_kernel<4, false>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((attn_split_kernel<kP256, false, kW256>), grid, dim3(kW256 * 64), 0, s, a);
  } else {
    if (a.split_keys <= 64)
      hipLaunchKernelGGL((attn_split_kernel<2, true>), grid, dim3(256), 0, s, a);
    else if (a.split_keys <= 128)
      hipLaunchKernelGGL((attn_split_kernel<4, true>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((attn_split_kernel<kP256, true, kW256>), grid, dim3(kW256 * 64), 0, s, a);
  }
  return fw_check_launch("attention split");
}

// Merges the split results of one head; splits with l == 0 are empty and skipped.
__global__ void __launch_bounds__(64) attn_combine_kernel(AttnArgs a, int nsplit) {
  const int head = blockIdx.x, d = threadIdx.x;
  const float* pm = a.part_m + head * nsplit;
  const float* pl = a.part_l + head * nsplit;
  const float* pa = a.part_acc + static_cast<size_t>(head) * nsplit * kHeadDim;
  float m = -INFINITY;
  for (int s = 0; s < nsplit; ++s) m = fmaxf(m, pm[s]);
  float num = 0.f, den = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    if (pl[s] > 0.f) {
      const float wgt = __expf(pm[s] - m);
      num = fmaf(pa[s * kHeadDim + d], wgt, num);
      den = fmaf(pl[s], wgt, den);
    }
  }
  a.out[head * kHeadDim + d] = f2h(num / den);
}

// ------------------------------------------------------------------------------------------
// Single-launch decode attention: one 1024-thread block (16 waves) per head covers every key, so
// the split partials never leave the CU (no workspace, no cross-block synchronisation). Keys are
// dealt to the 16 waves in equal multiples of 8; each wave issues all of its K and V loads at once
// (up to 12 passes x 8 keys = 96 keys, 24 x 16 B per lane in flight), then scores (fp32, scale after
// the dot), takes its local max/exp-sum/P.V, and the 16 wave partials are merged through LDS
// exactly like the split-K combine. Longer sequences run in rounds of 1536 keys with an online
// merge per wave. Self mode: the block writes k_new/v_new into row pos and uses them for key pos.
// ------------------------------------------------------------------------------------------
constexpr int kHeadWaves = 16, kHeadMaxPass = 12;
constexpr int kHeadRoundKeys = kHeadWaves * kHeadMaxPass * 8;

__global__ void __launch_bounds__(kHeadWaves * 64) attn_head_kernel(AttnArgs a) {
  __shared__ float wm[kHeadWaves], wl[kHeadWaves];
  __shared__ float wacc[kHeadWaves][kHeadDim];
  const int head = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int pos = attn_pos(a);
  const int len = a.len_state ? pos + 1 : a.max_len;
  const size_t hoff = static_cast<size_t>(head) * a.max_len * kHeadDim;
  _Float16* kh = a.k + hoff;
  _Float16* vh = a.v + hoff;
  const uint4* kn = a.k_new ? reinterpret_cast<const uint4*>(a.k_new + head * kHeadDim) : nullptr;
  const uint4* vn = a.v_new ? reinterpret_cast<const uint4*>(a.v_new + head * kHeadDim) : nullptr;
  if (kn && tid < 16) {
    if (tid < 8)
      reinterpret_cast<uint4*>(kh + static_cast<size_t>(pos) * kHeadDim)[tid] = kn[tid];
    else
      reinterpret_cast<uint4*>(vh + static_cast<size_t>(pos) * kHeadDim)[tid - 8] = vn[tid - 8];
  }
  const int ks = lane >> 3, c = lane & 7;
  const uint4 qc = reinterpret_cast<const uint4*>(a.q + head * kHeadDim)[c];

  float m_run = -INFINITY, l_run = 0.f, acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = 0.f;
  for (int base = 0; base < len; base += kHeadRoundKeys) {
    const int n_round = min(kHeadRoundKeys, len - base);
    const int per_wave = ((n_round + kHeadWaves * 8 - 1) / (kHeadWaves * 8)) * 8;  // multiple of 8
    const int w0 = base + wave * per_wave;
    const int w1 = min(w0 + per_wave, base + n_round);
    uint4 kr[kHeadMaxPass], vr[kHeadMaxPass];
#pragma unroll
    for (int p = 0; p < kHeadMaxPass; ++p) {
      const int j = w0 + p * 8 + ks;
      kr[p] = vr[p] = make_uint4(0, 0, 0, 0);
      if (j < w1) {
        const bool fresh = kn && j == pos;
        kr[p] = fresh ? kn[c] : reinterpret_cast<const uint4*>(kh + static_cast<size_t>(j) * kHeadDim)[c];
        vr[p] = fresh ? vn[c] : reinterpret_cast<const uint4*>(vh + static_cast<size_t>(j) * kHeadDim)[c];
      }
    }
    float s[kHeadMaxPass];
    float mx = -INFINITY;
#pragma unroll
    for (int p = 0; p < kHeadMaxPass; ++p) {
      const int j = w0 + p * 8 + ks;
      s[p] = group_sum<8>(dot8(kr[p], qc, 0.f)) * a.scale;
      if (j >= w1) s[p] = -INFINITY;
      mx = fmaxf(mx, s[p]);
    }
    mx = group_max<64>(mx);
    if (mx == -INFINITY) continue;  // this wave has no keys in this round (wave-uniform)
    const float m_new = fmaxf(m_run, mx);
    const float corr = __expf(m_run - m_new);
    float psum = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] *= corr;
#pragma unroll
    for (int p = 0; p < kHeadMaxPass; ++p) {
      const float pj = __expf(s[p] - m_new);  // 0 for masked keys
      psum += pj;
      const h2v* v2 = reinterpret_cast<const h2v*>(&vr[p]);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        acc[2 * t] = fmaf(pj, h2f(v2[t].x), acc[2 * t]);
        acc[2 * t + 1] = fmaf(pj, h2f(v2[t].y), acc[2 * t + 1]);
      }
    }
    // psum is replicated over the 8 lanes of a key group: sum one lane per group
    psum = xor_add<32>(xor_add<16>(xor_add<8>(psum)));
    l_run = l_run * corr + psum;
    m_run = m_new;
  }
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    acc[t] = xor_add<32>(xor_add<16>(xor_add<8>(acc[t])));
  }
  if (lane == 0) {
    wm[wave] = m_run;
    wl[wave] = l_run;
  }
  if (ks == 0) {
#pragma unroll
    for (int t = 0; t < 8; ++t) wacc[wave][c * 8 + t] = acc[t];
  }
  __syncthreads();
  if (tid < kHeadDim) {
    float m = -INFINITY;
#pragma unroll
    for (int w = 0; w < kHeadWaves; ++w) m = fmaxf(m, wm[w]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < kHeadWaves; ++w) {
      if (wl[w] > 0.f) {
        const float wgt = __expf(wm[w] - m);
        num = fmaf(wacc[w][tid], wgt, num);
        den = fmaf(wl[w], wgt, den);
      }
    }
    a.out[head * kHeadDim + tid] = f2h(num / den);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace fw

using namespace fw;

#define FW_REQUIRE(cond, ...)                         \
  do {                                                \
    if (!(cond)) return fw_fail(FW_EINVAL, __VA_ARGS__); \
  } while (0)

extern "C" int fw_lm_head_argmax(const void* y, const void* w, const uint8_t* suppress, int vocab, int hidden,
                                 uint64_t* best, hipStream_t stream) {
  FW_REQUIRE(y && w && suppress && best, "lm_head_argmax: null pointer");
  FW_REQUIRE(hidden == kHidden, "hidden size must be %d", kHidden);
  FW_REQUIRE(vocab > 0, "vocab must be positive");
  FW_REQUIRE(aligned16(y) && aligned16(w), "lm_head_argmax: y and w must be 16-byte aligned");
  const int grid = lm_head_grid(vocab);
  hipLaunchKernelGGL(lm_head_kernel<false>, dim3(grid), dim3(kLmNW * 64), 0, stream, static_cast<const _Float16*>(y),
                     LnArgs{}, static_cast<const _Float16*>(w), suppress, vocab,
                     reinterpret_cast<unsigned long long*>(best));
  return fw_check_launch("lm_head_argmax");
}

extern "C" int fw_lm_head_argmax_fused(const void* h, const void* x, const void* gamma, const void* beta, float eps,
                                       const void* w, const uint8_t* suppress, int vocab, int hidden, uint64_t* best,
                                       int64_t* tokens, int64_t* state, int64_t* cur, int max_pos,
                                       hipStream_t stream) {
  FW_REQUIRE(h && gamma && beta && w && suppress && best, "lm_head_argmax_fused: null pointer");
  const bool finalize = tokens || state || cur;
  FW_REQUIRE(!finalize || (tokens && state && cur), "lm_head_argmax_fused: tokens, state and cur must be given together");
  FW_REQUIRE(hidden == kHidden, "hidden size must be %d", kHidden);
  FW_REQUIRE(vocab > 0 && max_pos > 0, "vocab and max_pos must be positive");
  FW_REQUIRE(aligned16(w), "lm_head_argmax_fused: w must be 16-byte aligned");
  const int grid = lm_head_grid(vocab);
  LnArgs ln{static_cast<const _Float16*>(h), static_cast<const _Float16*>(x), nullptr,
            static_cast<const _Float16*>(gamma), static_cast<const _Float16*>(beta), eps, nullptr, nullptr,
            nullptr, nullptr, 0, 0};
  hipLaunchKernelGGL(lm_head_kernel<true>, dim3(grid), dim3(kLmNW * 64), 0, stream, nullptr, ln,
                     static_cast<const _Float16*>(w), suppress, vocab, reinterpret_cast<unsigned long long*>(best));
  int rc = fw_check_launch("lm_head_argmax_fused");
  if (rc != FW_OK || !finalize) return rc;
  FinArgs fin{tokens, state, cur, max_pos};
  hipLaunchKernelGGL(argmax_finalize_kernel, dim3(1), dim3(1), 0, stream, reinterpret_cast<unsigned long long*>(best),
                     fin);
  return fw_check_launch("lm_head_argmax_fused finalize");
}

extern "C" int fw_lm_head_q8_pack(const void* w, int vocab, int hidden, void* wq, float* meta, hipStream_t stream) {
  FW_REQUIRE(w && wq && meta, "lm_head_q8_pack: null pointer");
  FW_REQUIRE(hidden == kHidden, "hidden size must be %d", kHidden);
  FW_REQUIRE(vocab > 0, "vocab must be positive");
  FW_REQUIRE((reinterpret_cast<uintptr_t>(meta) & 7u) == 0, "lm_head_q8_pack: meta must be 8-byte aligned");
  hipLaunchKernelGGL(lm_q8_pack_kernel, dim3((vocab + 3) / 4), dim3(256), 0, stream, static_cast<const _Float16*>(w),
                     vocab, static_cast<int8_t*>(wq), reinterpret_cast<float2*>(meta));
  return fw_check_launch("lm_head_q8_pack");
}

extern "C" int fw_lm_head_argmax_q8(const void* h, const void* x, const void* gamma, const void* beta, float eps,
                                    const void* w, const void* wq, const float* meta, const uint8_t* suppress,
                                    int vocab, int hidden, uint64_t* best, int64_t* tokens, int64_t* state,
                                    int64_t* cur, int max_pos, hipStream_t stream) {
  FW_REQUIRE(h && gamma && beta && w && wq && meta && suppress && best, "lm_head_argmax_q8: null pointer");
  const bool finalize = tokens || state || cur;
  FW_REQUIRE(!finalize || (tokens && state && cur), "lm_head_argmax_q8: tokens, state and cur must be given together");
  FW_REQUIRE(hidden == kHidden, "hidden size must be %d", kHidden);
  FW_REQUIRE(vocab > 0 && max_pos > 0, "vocab and max_pos must be positive");
  FW_REQUIRE(aligned16(w) && aligned16(wq) && (reinterpret_cast<uintptr_t>(meta) & 7u) == 0,
             "lm_head_argmax_q8: w and wq must be 16-byte aligned, meta 8-byte aligned");
  LnArgs ln{static_cast<const _Float16*>(h), static_cast<const _Float16*>(x), nullptr,
            static_cast<const _Float16*>(gamma), static_cast<const _Float16*>(beta), eps, nullptr, nullptr,
            nullptr, nullptr, 0, 0};
  hipLaunchKernelGGL(lm_head_q8_kernel<true>, dim3(lm_head_q8_grid(vocab)), dim3(kLmNW * 64), 0, stream, nullptr, ln,
                     static_cast<const _Float16*>(w), static_cast<const int8_t*>(wq),
                     reinterpret_cast<const float2*>(meta), suppress, vocab,
                     reinterpret_cast<unsigned long long*>(best));
  int rc = fw_check_launch("lm_head_argmax_q8");
  if (rc != FW_OK || !finalize) return rc;
  FinArgs fin{tokens, state, cur, max_pos};
  hipLaunchKernelGGL(argmax_finalize_kernel, dim3(1), dim3(1), 0, stream, reinterpret_cast<unsigned long long*>(best),
                     fin);
  return fw_check_launch("lm_head_argmax_q8 finalize");
}

extern "C" int fw_argmax_finalize(uint64_t* best, int64_t* tokens, int64_t* state, int64_t* cur, int max_pos,
                                  hipStream_t stream) {
  FW_REQUIRE(best && tokens && state && cur, "argmax_finalize: null pointer");
  FW_REQUIRE(max_pos > 0, "max_pos must be positive");
  FinArgs fin{tokens, state, cur, max_pos};
  hipLaunchKernelGGL(argmax_finalize_kernel, dim3(1), dim3(1), 0, stream, reinterpret_cast<unsigned long long*>(best),
                     fin);
  return fw_check_launch("argmax_finalize");
}

static int attention_common(const void* q, void* k, void* v, void* out, const int64_t* len_state, const void* k_new,
                            const void* v_new, int heads, int max_len, AttnArgs* a) {
  FW_REQUIRE(q && k && v, "decode_attention: null pointer");
  FW_REQUIRE(heads > 0 && max_len > 0, "decode_attention: heads and max_len must be positive");
  FW_REQUIRE((k_new != nullptr) == (v_new != nullptr) && (k_new != nullptr) == (len_state != nullptr),
             "len_state, k_new and v_new must be given together");
  FW_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && (!k_new || (aligned16(k_new) && aligned16(v_new))),
             "decode_attention: q, k, v, k_new, v_new must be 16-byte aligned");
  *a = AttnArgs{static_cast<const _Float16*>(q), static_cast<_Float16*>(k), static_cast<_Float16*>(v),
                static_cast<const _Float16*>(k_new), static_cast<const _Float16*>(v_new), len_state, max_len,
                kSplitKeys, 0.f, nullptr, nullptr, nullptr, static_cast<_Float16*>(out), 0, 0};
  return FW_OK;
}

extern "C" int fw_decode_attention(const void* q, void* k, void* v, void* out, const int64_t* len_state,
                                   const void* k_new, const void* v_new, int heads, int max_len, float* part_m,
                                   float* part_l, float* part_acc, int64_t ws_slots, float scale, hipStream_t stream) {
  FW_REQUIRE(out, "decode_attention: null out");
  AttnArgs a;
  int rc = attention_common(q, k, v, out, len_state, k_new, v_new, heads, max_len, &a);
  if (rc != FW_OK) return rc;
  FW_REQUIRE(part_m && part_l && part_acc, "decode_attention: null workspace");
  const int nsplit = (max_len + kSplitKeys - 1) / kSplitKeys;
  FW_REQUIRE(ws_slots >= static_cast<int64_t>(heads) * nsplit, "workspace too small for %d splits", nsplit);
  a.scale = scale;
  a.part_m = part_m;
  a.part_l = part_l;
  a.part_acc = part_acc;
  rc = launch_attn_split(a, nsplit, heads, stream);
  if (rc != FW_OK) return rc;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(heads), dim3(kHeadDim), 0, stream, a, nsplit);
  return fw_check_launch("decode_attention combine");
}

extern "C" int fw_decode_attention_fused(const void* q, void* k, void* v, void* out, const int64_t* len_state,
                                         const void* k_new, const void* v_new, int heads, int max_len, float scale,
                                         hipStream_t stream) {
  FW_REQUIRE(out, "decode_attention_fused: null out");
  AttnArgs a;
  int rc = attention_common(q, k, v, out, len_state, k_new, v_new, heads, max_len, &a);
  if (rc != FW_OK) return rc;
  a.scale = scale;
  hipLaunchKernelGGL(attn_head_kernel, dim3(heads), dim3(kHeadWaves * 64), 0, stream, a);
  return fw_check_launch("decode_attention_fused");
}

extern "C" int fw_add_layernorm(void* h, const void* x, const void* gamma, const void* beta, void* y, int n, float eps,
                                hipStream_t stream) {
  FW_REQUIRE(h && gamma && beta && y, "add_layernorm: null pointer");
  FW_REQUIRE(n == kHidden, "hidden size must be %d", kHidden);
  FW_REQUIRE(aligned16(h) && aligned16(gamma) && aligned16(beta) && aligned16(y) && (!x || aligned16(x)),
             "add_layernorm: tensors must be 16-byte aligned");
  hipLaunchKernelGGL(add_layernorm_kernel, dim3(1), dim3(256), 0, stream, static_cast<_Float16*>(h),
                     static_cast<const _Float16*>(x), static_cast<const _Float16*>(gamma),
                     static_cast<const _Float16*>(beta), static_cast<_Float16*>(y), eps);
  return fw_check_launch("add_layernorm");
}

extern "C" int fw_final_layernorm(const void* h, const void* x, const void* gamma, const void* beta, void* y, int n,
                                  float eps, hipStream_t stream) {
  FW_REQUIRE(h && gamma && beta && y, "final_layernorm: null pointer");
  FW_REQUIRE(n == kHidden, "hidden size must be %d", kHidden);
  hipLaunchKernelGGL(final_layernorm_kernel, dim3(1), dim3(1024), 0, stream, static_cast<const _Float16*>(h),
                     static_cast<const _Float16*>(x), static_cast<const _Float16*>(gamma),
                     static_cast<const _Float16*>(beta), static_cast<_Float16*>(y), eps);
  return fw_check_launch("final_layernorm");
}

extern "C" int fw_embed(const int64_t* cur, const int64_t* state, const void* embed, const void* pos_embed, int vocab,
                        int max_pos, void* h, int hidden, hipStream_t stream) {
  FW_REQUIRE(cur && state && embed && pos_embed && h, "embed: null pointer");
  FW_REQUIRE(hidden == kHidden, "hidden size must be %d", kHidden);
  FW_REQUIRE(vocab > 0 && max_pos > 0, "vocab and max_pos must be positive");
  hipLaunchKernelGGL(embed_kernel, dim3(1), dim3(256), 0, stream, cur, state, static_cast<const _Float16*>(embed),
                     static_cast<const _Float16*>(pos_embed), vocab, max_pos, static_cast<_Float16*>(h));
  return fw_check_launch("embed");
}

static int gemv_impl(const void* x, const void* w, const void* bias, void* out, int n_out, int k_in, int act, int nv,
                     hipStream_t stream) {
  FW_REQUIRE(x && w && out, "gemv: null pointer");
  FW_REQUIRE(n_out > 0, "gemv: n_out must be positive");
  FW_REQUIRE(k_in == kHidden || k_in == 4 * kHidden, "gemv: k_in must be 1280 or 5120");
  FW_REQUIRE(act == FW_ACT_NONE || act == FW_ACT_GELU, "gemv: unknown activation %d", act);
  FW_REQUIRE(nv >= 1 && nv <= kMaxBatch, "gemv: nv must be in [1, %d]", kMaxBatch);
  FW_REQUIRE(aligned16(x) && aligned16(w), "gemv: x and w must be 16-byte aligned");
  const auto* xp = static_cast<const _Float16*>(x);
  const auto* wp = static_cast<const _Float16*>(w);
  const auto* bp = static_cast<const _Float16*>(bias);
  auto* op = static_cast<_Float16*>(out);
  const LnArgs ln{};
  const CombineArgs cb{};
  if (k_in == kHidden) {
    if (act == FW_ACT_GELU)
      dispatch_gemv_1280_batch<kModePlain, FW_ACT_GELU>(nv, xp, ln, cb, wp, bp, op, n_out, stream);
    else
      dispatch_gemv_1280_batch<kModePlain, FW_ACT_NONE>(nv, xp, ln, cb, wp, bp, op, n_out, stream);
  } else if (nv == 1) {
    if (act == FW_ACT_GELU)
      launch_gemv<4 * kHidden, FW_GK5120_NW, FW_GK5120_U, kModePlain, FW_ACT_GELU>(xp, ln, cb, wp, bp, op, n_out, stream);
    else
      launch_gemv<4 * kHidden, FW_GK5120_NW, FW_GK5120_U, kModePlain, FW_ACT_NONE>(xp, ln, cb, wp, bp, op, n_out, stream);
  } else {
    if (act == FW_ACT_GELU)
      launch_gemv_batch<4 * kHidden, FW_GK5120_NW, kModePlain, FW_ACT_GELU>(nv, xp, ln, cb, wp, bp, op, n_out, stream);
    else
      launch_gemv_batch<4 * kHidden, FW_GK5120_NW, kModePlain, FW_ACT_NONE>(nv, xp, ln, cb, wp, bp, op, n_out, stream);
  }
  return fw_check_launch("gemv");
}

extern "C" int fw_gemv(const void* x, const void* w, const void* bias, void* out, int n_out, int k_in, int act,
                       hipStream_t stream) {
  return gemv_impl(x, w, bias, out, n_out, k_in, act, 1, stream);
}

extern "C" int fw_gemv_batch(const void* x, const void* w, const void* bias, void* out, int n_out, int k_in, int act,
                             int nv, hipStream_t stream) {
  return gemv_impl(x, w, bias, out, n_out, k_in, act, nv, stream);
}

static int ln_gemv_impl(const void* h, const void* x, void* h_out, const void* gamma, const void* beta, float eps,
                        const int64_t* cur, const int64_t* state, const void* embed, const void* pos_embed, int vocab,
                        int max_pos, const void* w, const void* bias, void* out, int n_out, int k_in, int act, int nv,
                        hipStream_t stream) {
  FW_REQUIRE(gamma && beta && w && out, "ln_gemv: null pointer");
  FW_REQUIRE(nv >= 1 && nv <= kMaxBatch, "ln_gemv: nv must be in [1, %d]", kMaxBatch);
  FW_REQUIRE(k_in == kHidden, "ln_gemv: k_in must be %d", kHidden);
  FW_REQUIRE(n_out > 0, "ln_gemv: n_out must be positive");
  FW_REQUIRE(act == FW_ACT_NONE || act == FW_ACT_GELU, "ln_gemv: unknown activation %d", act);
  FW_REQUIRE(aligned16(w), "ln_gemv: w must be 16-byte aligned");
  if (cur) {
    FW_REQUIRE(state && embed && pos_embed && vocab > 0 && max_pos > 0, "ln_gemv: embedding mode needs state, tables");
  } else {
    FW_REQUIRE(h != nullptr, "ln_gemv: null h");
    FW_REQUIRE(h_out != h, "ln_gemv: h_out must not alias h");
  }
  LnArgs ln{static_cast<const _Float16*>(h), static_cast<const _Float16*>(x), static_cast<_Float16*>(h_out),
            static_cast<const _Float16*>(gamma), static_cast<const _Float16*>(beta), eps, cur, state,
            static_cast<const _Float16*>(embed), static_cast<const _Float16*>(pos_embed), vocab, max_pos};
  const auto* wp = static_cast<const _Float16*>(w);
  const auto* bp = static_cast<const _Float16*>(bias);
  auto* op = static_cast<_Float16*>(out);
  const CombineArgs cb{};
  if (act == FW_ACT_GELU)
    dispatch_gemv_1280_batch<kModeLn, FW_ACT_GELU>(nv, nullptr, ln, cb, wp, bp, op, n_out, stream);
  else
    dispatch_gemv_1280_batch<kModeLn, FW_ACT_NONE>(nv, nullptr, ln, cb, wp, bp, op, n_out, stream);
  return fw_check_launch("ln_gemv");
}

extern "C" int fw_ln_gemv(const void* h, const void* x, void* h_out, const void* gamma, const void* beta, float eps,
                          const int64_t* cur, const int64_t* state, const void* embed, const void* pos_embed,
                          int vocab, int max_pos, const void* w, const void* bias, void* out, int n_out, int k_in,
                          int act, hipStream_t stream) {
  return ln_gemv_impl(h, x, h_out, gamma, beta, eps, cur, state, embed, pos_embed, vocab, max_pos, w, bias, out, n_out,
                      k_in, act, 1, stream);
}

extern "C" int fw_ln_gemv_batch(const void* h, const void* x, void* h_out, const void* gamma, const void* beta,
                                float eps, const int64_t* cur, const int64_t* state, const void* embed,
                                const void* pos_embed, int vocab, int max_pos, const void* w, const void* bias,
                                void* out, int n_out, int k_in, int act, int nv, hipStream_t stream) {
  return ln_gemv_impl(h, x, h_out, gamma, beta, eps, cur, state, embed, pos_embed, vocab, max_pos, w, bias, out, n_out,
                      k_in, act, nv, stream);
}

static int attention_split_impl(const void* q, void* k, void* v, const int64_t* len_state, const void* k_new,
                                const void* v_new, int heads, int max_len, int split_keys, float* part_m,
                                float* part_l, float* part_acc, int64_t ws_slots, float scale, int nq, int q_stride,
                                int kv_stride, hipStream_t stream) {
  AttnArgs a;
  int rc = attention_common(q, k, v, nullptr, len_state, k_new, v_new, heads, max_len, &a);
  if (rc != FW_OK) return rc;
  FW_REQUIRE(part_m && part_l && part_acc, "attention_split: null workspace");
  FW_REQUIRE(split_keys >= 8 && split_keys <= 256 && split_keys % 8 == 0,
             "split_keys must be a multiple of 8 in [8, 256]");
  FW_REQUIRE(nq >= 1 && nq <= kMaxBatch, "attention_split: nq must be in [1, %d]", kMaxBatch);
  if (nq > 1) {
    FW_REQUIRE(q_stride >= heads * kHeadDim && q_stride % 8 == 0,
               "attention_split: q_stride must be a multiple of 8 and at least heads * 64");
    FW_REQUIRE(!k_new || (kv_stride >= heads * kHeadDim && kv_stride % 8 == 0),
               "attention_split: kv_stride must be a multiple of 8 and at least heads * 64");
  }
  const int nsplit = (max_len + split_keys - 1) / split_keys;
  FW_REQUIRE(ws_slots >= static_cast<int64_t>(nq) * heads * nsplit, "workspace too small for %d x %d splits", nq,
             nsplit);
  a.out = nullptr;
  a.split_keys = split_keys;
  a.scale = scale;
  a.part_m = part_m;
  a.part_l = part_l;
  a.part_acc = part_acc;
  a.q_stride = nq > 1 ? q_stride : 0;
  a.kv_stride = nq > 1 && k_new ? kv_stride : 0;
  return launch_attn_split(a, nsplit, heads, stream, nq);
}

extern "C" int fw_attention_split(const void* q, void* k, void* v, const int64_t* len_state, const void* k_new,
                                  const void* v_new, int heads, int max_len, int split_keys, float* part_m,
                                  float* part_l, float* part_acc, int64_t ws_slots, float scale, hipStream_t stream) {
  return attention_split_impl(q, k, v, len_state, k_new, v_new, heads, max_len, split_keys, part_m, part_l, part_acc,
                              ws_slots, scale, 1, 0, 0, stream);
}

extern "C" int fw_attention_split_batch(const void* q, void* k, void* v, const int64_t* len_state, const void* k_new,
                                        const void* v_new, int heads, int max_len, int split_keys, float* part_m,
                                        float* part_l, float* part_acc, int64_t ws_slots, float scale, int nq,
                                        int q_stride, int kv_stride, hipStream_t stream) {
  return attention_split_impl(q, k, v, len_state, k_new, v_new, heads, max_len, split_keys, part_m, part_l, part_acc,
                              ws_slots, scale, nq, q_stride, kv_stride, stream);
}

static int attn_out_gemv_impl(const float* part_m, const float* part_l, const float* part_acc, int64_t ws_slots,
                              const int64_t* len_state, int heads, int max_len, int split_keys, const void* w,
                              const void* bias, void* out, int n_out, int nv, hipStream_t stream) {
  FW_REQUIRE(part_m && part_l && part_acc && w && out, "attn_out_gemv: null pointer");
  FW_REQUIRE(nv >= 1 && nv <= kMaxBatch, "attn_out_gemv: nv must be in [1, %d]", kMaxBatch);
  FW_REQUIRE(heads * kHeadDim == kHidden, "attn_out_gemv: heads * 64 must be %d", kHidden);
  FW_REQUIRE(max_len > 0 && split_keys >= 8 && n_out > 0, "attn_out_gemv: bad sizes");
  FW_REQUIRE(aligned16(w), "attn_out_gemv: w must be 16-byte aligned");
  const int nsplit = (max_len + split_keys - 1) / split_keys;
  FW_REQUIRE(nsplit <= kMaxCombineSplits && heads <= kMaxCombineHeads,
             "attn_out_gemv: at most %d splits (got %d) and %d heads", kMaxCombineSplits, nsplit, kMaxCombineHeads);
  FW_REQUIRE(ws_slots >= static_cast<int64_t>(nv) * heads * nsplit, "attn_out_gemv: workspace too small");
  const CombineArgs cb{part_m, part_l, part_acc, len_state, max_len, split_keys, nsplit, heads, 0};
  const auto* wp = static_cast<const _Float16*>(w);
  const auto* bp = static_cast<const _Float16*>(bias);
  auto* op = static_cast<_Float16*>(out);
  if (nv == 1)
    launch_gemv<kHidden, FW_CMB_NW, 1, kModeCombine, FW_ACT_NONE>(nullptr, LnArgs{}, cb, wp, bp, op, n_out, stream);
  else
    launch_gemv_batch<kHidden, FW_CMB_NW, kModeCombine, FW_ACT_NONE>(nv, nullptr, LnArgs{}, cb, wp, bp, op, n_out,
                                                                     stream);
  return fw_check_launch("attn_out_gemv");
}

extern "C" int fw_attn_out_gemv(const float* part_m, const float* part_l, const float* part_acc, int64_t ws_slots,
                                const int64_t* len_state, int heads, int max_len, int split_keys, const void* w,
                                const void* bias, void* out, int n_out, hipStream_t stream) {
  return attn_out_gemv_impl(part_m, part_l, part_acc, ws_slots, len_state, heads, max_len, split_keys, w, bias, out,
                            n_out, 1, stream);
}

extern "C" int fw_attn_out_gemv_batch(const float* part_m, const float* part_l, const float* part_acc,
                                      int64_t ws_slots, const int64_t* len_state, int heads, int max_len,
                                      int split_keys, const void* w, const void* bias, void* out, int n_out, int nv,
                                      hipStream_t stream) {
  return attn_out_gemv_impl(part_m, part_l, part_acc, ws_slots, len_state, heads, max_len, split_keys, w, bias, out,
                            n_out, nv, stream);
}

// ------------------------------------------------------------------------------------------
// fw_decode_attention without a workspace argument, for callers that cannot allocate. The split
// partials live in `scratch`, a device array of this library: each GPU holds its own copy until
// the process ends. Its address on a device is looked up once (hipGetSymbolAddress, with that device
// current) and kept; the kernels are given that address, never the host-side symbol. Every call on
// one GPU shares the array, so calls that overlap on one GPU race. Nothing in it has to start at
// zero: the split launch writes every (m, l) slot the combine reads (m = -inf, l = 0 for an empty
// split), and the combine reads the value sums only of splits with l > 0.
// ------------------------------------------------------------------------------------------
static_assert(FW_NOALLOC_ATTN_SLOTS > 0 && kHeadDim == 64, "static workspace layout");
static __device__ __align__(256) float scratch[FW_NOALLOC_ATTN_SLOTS * (2 + 64)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
std::atomic<float*> g_scratch_ptr[kMaxDevices];

int noalloc_scratch(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fw_fail(FW_EHIP, "decode_attention_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  FW_REQUIRE(dev >= 0 && dev < kMaxDevices, "decode_attention_noalloc: device %d out of range", dev);
  float* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      void* addr = nullptr;
      e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || addr == nullptr)
        return fw_fail(FW_EHIP, "decode_attention_noalloc: hipGetSymbolAddress on device %d: %s", dev,
                       hipGetErrorString(e));
      p = static_cast<float*>(addr);
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return FW_OK;
}
}  // namespace

extern "C" int fw_decode_attention_noalloc(const void* q, void* k, void* v, void* out, const int64_t* len_state,
                                           const void* k_new, const void* v_new, int heads, int max_len, float scale,
                                           hipStream_t stream) {
  FW_REQUIRE(out, "decode_attention_noalloc: null out");
  AttnArgs a;
  int rc = attention_common(q, k, v, out, len_state, k_new, v_new, heads, max_len, &a);
  if (rc != FW_OK) return rc;
  const int nsplit = (max_len + kSplitKeys - 1) / kSplitKeys;
  FW_REQUIRE(static_cast<int64_t>(heads) * nsplit <= FW_NOALLOC_ATTN_SLOTS,
             "decode_attention_noalloc: heads * ceil(max_len / %d) = %lld exceeds the %d slots of the static "
             "workspace",
             kSplitKeys, static_cast<long long>(heads) * nsplit, FW_NOALLOC_ATTN_SLOTS);
  float* ws = nullptr;
  rc = noalloc_scratch(&ws);
  if (rc != FW_OK) return rc;
  a.scale = scale;
  a.part_m = ws;
  a.part_l = ws + FW_NOALLOC_ATTN_SLOTS;
  a.part_acc = ws + 2 * FW_NOALLOC_ATTN_SLOTS;
  rc = launch_attn_split(a, nsplit, heads, stream);
  if (rc != FW_OK) return rc;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(heads), dim3(kHeadDim), 0, stream, a, nsplit);
  return fw_check_launch("decode_attention_noalloc combine");
}
