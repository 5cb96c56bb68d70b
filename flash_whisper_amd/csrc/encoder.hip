// Whisper encoder kernels for gfx950: an MFMA GEMM with fused epilogues (also used as an
// implicit-GEMM conv1d and for the decoder cross K/V projection) and a row LayerNorm; the encoder
// self-attention is in attention_enc.hip. Semantics follow HF WhisperEncoder.forward in fp16
// (transformers models/whisper/modeling_whisper.py:592-648, layer :379-414, attention :284-358):
// every op output is rounded to fp16, accumulation is fp32.
#include "lds_pipe.h"

namespace fw {
namespace {

// ------------------------------------------------------------------------------------------
// GEMM: out[m, n] = epi(sum_k A[m, k] * W[n, k]).  Block tile BM x 128 x 64 with BM in
// {256, 192, 128, 64}; waves in a (BM / 64 or 2) x 2 arrangement, each wave a (64 or 32) x 64 tile of
// v_mfma_f32_32x32x16_f16 products (192-row tiles: 2 x 4 waves of 96 x 32; 64-row tiles: 2 x 4 waves
// of 32 x 32).
//  - LDS: one [rows][64] fp16 tile per operand and stage, 8 x 16-byte chunks per row, chunk c of
//    row r stored in slot swz_slot(r, c) = c ^ ((r >> 1) & 7), so the 16 rows a 16-lane group reads
//    for one MFMA operand cover all 64 banks (conflict-free ds_read_b128).
//  - Epilogues: bias, GELU (erfc by a fitted exponent polynomial, one fp16 ulp of the exact-erf GELU at most),
//    residual, fp16 clamp, the q scale, the cross K/V scatter and the transposed-V store.
//  - Plain GEMMs (gemm_dma_kernel): global -> LDS copies into a ring of stages, operand fragments
//    double-buffered in registers (see the pipeline notes above that kernel).
//  - Implicit-GEMM conv: a 64-wide k stage of A row m is 64 contiguous channels of input row
//    m * stride + tap - 1, so long-k convs use the same direct-to-LDS pipeline (padding rows copy
//    from a zero row); short-k convs gather the A tile through registers (gemm_kernel: two staging
//    sets, two LDS buffers).
//  - Tile order: hardware deals blocks round-robin over the 8 XCDs; the block id is remapped so each
//    XCD works on its own part of the tile grid and its L2 sees only that part's operand panels.
// MFMA 32x32x16 f16 operand layout (lane l, g = l / 32):
//   A: lane holds A[l % 32][8g .. 8g + 7]      B: lane holds B[8g .. 8g + 7][l % 32]
//   C: acc[r] = C[8 (r / 4) + 4 g + (r % 4)][l % 32], r = 0 .. 15
// ------------------------------------------------------------------------------------------
constexpr int kBN = 128, kBK = 64;
constexpr int kEpiCrossKV = 100;  // internal epilogue: scatter into [layers, 2, heads, t, 64]
// Internal epilogue of the encoder q/k/v projection: q columns scaled as FW_EPI_SCALE_Q, k columns
// stored as they are, v columns stored transposed into vt (the attention kernel's V layout).
constexpr int kEpiQkvVt = 101;
// Internal epilogue of the split-k products: split s (blockIdx.x / tiles) covers k in [s k, (s + 1) k)
// and stores its fp32 sums to part[s][m][n]; the row kernel that follows adds the splits.
constexpr int kEpiPartial = 102;

struct GemmArgs {
  const _Float16* a;
  int lda;
  const _Float16* w;
  int ldw;
  const _Float16* bias;
  _Float16* out;
  int ldo;
  const _Float16* res;
  int ldr;
  int m, n, k;
  int q_cols;
  // implicit conv1d (k = 3, pad 1): a is x[t_in, c_in]; row m, column kk = tap * c_in + c reads
  // x[m * stride + tap - 1, c], zero outside [0, t_in).
  int conv_stride;  // 0: plain GEMM
  int t_in, c_in;
  // cross K/V scatter
  int heads, t_len;
  // q/k/v projection: transposed V, [heads * 64][vt_pad]
  _Float16* vt;
  int vt_pad;
  // XCD tile grouping (0: none): the 8 XCDs split the tile grid into xm x xn rectangles
  int xm, xn;
  // split-k products (kEpiPartial): number of splits and the fp32 partial sums [splits][m][n]
  int splits;
  float* part;
};

// Block -> output tile. Hardware deals workgroups round-robin over the 8 XCDs (block b runs on XCD
// b % 8), each with its own L2. With a grouping, XCD x owns one (ntm / xm) x (ntn / xn) rectangle of
// the tile grid, so each XCD fetches only its slices of A and W. Otherwise each XCD takes a contiguous
// run of row-major tiles (the tail beyond a multiple of 8 keeps its id). Both maps are bijective.
template <int BM>
__device__ __forceinline__ void tile_origin(const GemmArgs& g, int& m0, int& n0) {
  const int ntn = g.n / kBN, ntm = (g.m + BM - 1) / BM;
  const int bid = g.splits > 1 ? static_cast<int>(blockIdx.x) % (ntn * ntm) : static_cast<int>(blockIdx.x);
  int tm, tn;
  if (g.xm) {
    const int xcd = bid & 7, local = bid >> 3, mr = ntm / g.xm, nr = ntn / g.xn;
    tm = (xcd / g.xn) * mr + local % mr;
    tn = (xcd % g.xn) * nr + local / mr;
  } else {
    const int ntiles = ntn * ntm, full = (ntiles / 8) * 8;
    const int tile = bid < full ? (bid % 8) * (full / 8) + bid / 8 : bid;
    tm = tile / ntn;
    tn = tile % ntn;
  }
  m0 = tm * BM;
  n0 = tn * kBN;
}

constexpr bool epi_reads_res(int epi) {
  return epi == FW_EPI_BIAS_RESID || epi == FW_EPI_BIAS_RESID_CLAMP || epi == FW_EPI_BIAS_GELU_POS;
}

// GELU(x) = x Phi(x) with Phi(x) = erfc(-x / sqrt 2) / 2, written as in Press et al., Numerical
// Recipes in C (2nd ed.), 6.2 ("erfcc"): with z = |x| / sqrt 2 and t = 1 / (1 + z / 2),
//   erfc(z) / 2 = t 2^(Q(t) - z^2 log2 e),
// where Q(t) = log2(erfc(z) / (2 t)) + z^2 log2 e is smooth in t. Q here is our own degree-7 fit
// (near-minimax by iteratively reweighted least squares against float64 erfc on t in [0.3, 1], i.e.
// z <= 4.67; max |error| 4.0e-7 in log2 units, so erfc carries a relative error below 3e-7), with the
// 1/2 and the log2 e scaling folded into the coefficients. On both tails the result is accurate in
// relative terms; rounded to fp16 it equals the exact-erf GELU on all but 7 of the finite fp16
// inputs, which are one ulp off (the same count as the Numerical Recipes coefficients, which cost
// two more FMAs and three more scalings per element; the fc1 epilogue is bound by VALU issue).
// Beyond z = 4.67 the GELU underflows fp16 on the negative side and equals x on the positive side.
__device__ __forceinline__ float gelu_enc(float x) {
  const float t = __builtin_amdgcn_rcpf(fmaf(fabsf(x), 0.35355339059327376f, 1.0f));
  float q = -0.19670111f;
  q = fmaf(t, q, 0.74583995f);
  q = fmaf(t, q, -0.79930210f);
  q = fmaf(t, q, -0.15935127f);
  q = fmaf(t, q, 0.34100536f);
  q = fmaf(t, q, 0.42959806f);
  q = fmaf(t, q, 1.46661794f);
  q = fmaf(t, q, -2.82770705f);
  const float c = t * __builtin_amdgcn_exp2f(fmaf(x * x, -0.72134752f, q));  // Phi(-|x|)
  return x * (x >= 0.0f ? 1.0f - c : c);
}

// Output value before the final fp16 rounding; `res` is the residual / position operand of the
// epilogues that read one.
__device__ __forceinline__ float epilogue_apply(int epi, float acc, float b, float res, int col, int q_cols) {
  float v = round_h(acc + b);
  switch (epi) {
    case FW_EPI_BIAS_GELU:
      v = gelu_enc(v);
      break;
    case FW_EPI_BIAS_RESID:
      v = res + v;
      break;
    case FW_EPI_BIAS_RESID_CLAMP: {
      v = round_h(res + v);
      const float c = 65504.0f - 1000.0f;
      v = fminf(fmaxf(v, -c), c);
      break;
    }
    case FW_EPI_BIAS_GELU_POS:
      v = round_h(gelu_enc(v)) + res;
      break;
    case FW_EPI_SCALE_Q:
    case kEpiQkvVt:
      if (col < q_cols) v = v * 0.125f;
      break;
    default:
      break;
  }
  return v;
}

__device__ __forceinline__ float epilogue_value(int epi, float acc, float b, const GemmArgs& g, int row, int col) {
  const float res = epi_reads_res(epi) ? h2f(g.res[static_cast<size_t>(row) * g.ldr + col]) : 0.f;
  return epilogue_apply(epi, acc, b, res, col, g.q_cols);
}


template <int BM>
struct GemmStage {
  static constexpr int kA = BM * 8 / 256;   // 16-byte A chunks per thread per stage
  static constexpr int kB = kBN * 8 / 256;  // 16-byte B chunks per thread per stage
  u32x4 a[kA];
  u32x4 b[kB];
};

template <int BM, bool CONV>
__device__ __forceinline__ void gemm_load(const GemmArgs& g, int m0, int n0, int k0, int tid, GemmStage<BM>& st) {
#pragma unroll
  for (int i = 0; i < GemmStage<BM>::kA; ++i) {
    const int c = tid + 256 * i;
    const int row = c >> 3, kc = (c & 7) * 8;
    const int gm = m0 + row;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (gm < g.m) {
      if constexpr (CONV) {
        const int kk = k0 + kc;
        const int tap = kk / g.c_in, ch = kk - tap * g.c_in;
        const int src = gm * g.conv_stride + tap - 1;
        if (src >= 0 && src < g.t_in) v = *reinterpret_cast<const u32x4*>(g.a + static_cast<size_t>(src) * g.c_in + ch);
      } else {
        v = *reinterpret_cast<const u32x4*>(g.a + static_cast<size_t>(gm) * g.lda + k0 + kc);
      }
    }
    st.a[i] = v;
  }
#pragma unroll
  for (int i = 0; i < GemmStage<BM>::kB; ++i) {
    const int c = tid + 256 * i;
    const int row = c >> 3, kc = (c & 7) * 8;
    st.b[i] = *reinterpret_cast<const u32x4*>(g.w + static_cast<size_t>(n0 + row) * g.ldw + k0 + kc);
  }
}

template <int BM>
__device__ __forceinline__ void gemm_store(u32x4* As, u32x4* Bs, int tid, const GemmStage<BM>& st) {
#pragma unroll
  for (int i = 0; i < GemmStage<BM>::kA; ++i) {
    const int c = tid + 256 * i;
    As[swz(c >> 3, c & 7)] = st.a[i];
  }
#pragma unroll
  for (int i = 0; i < GemmStage<BM>::kB; ++i) {
    const int c = tid + 256 * i;
    Bs[swz(c >> 3, c & 7)] = st.b[i];
  }
}

template <int kTM, int kTN>
__device__ __forceinline__ void gemm_mma(const u32x4* As, const u32x4* Bs, int wm, int wn, int lr, int lg,
                                         f16v (&acc)[kTM][kTN]) {
#pragma unroll
  for (int s = 0; s < kBK / 16; ++s) {
    h8v av[kTM], bv[kTN];
#pragma unroll
    for (int i = 0; i < kTM; ++i) av[i] = __builtin_bit_cast(h8v, As[swz(wm + 32 * i + lr, 2 * s + lg)]);
#pragma unroll
    for (int j = 0; j < kTN; ++j) bv[j] = __builtin_bit_cast(h8v, Bs[swz(wn + 32 * j + lr, 2 * s + lg)]);
#pragma unroll
    for (int i = 0; i < kTM; ++i)
#pragma unroll
      for (int j = 0; j < kTN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
  }
}

// MFMA operand fragments of one 64-wide k stage for a wave: A rows wm + 32 i + lane % 32, B rows
// wn + 32 j + lane % 32, k-step s covering k 16 s .. 16 s + 15.
template <int kTM, int kTN>
struct Frags {
  h8v a[kBK / 16][kTM];
  h8v b[kBK / 16][kTN];
};

// Byte offsets, within one ring stage (A tile, then the B tile at BM * 128 bytes), of a lane's
// fragments for each k-step s. Rows wm + 32 i + lr and wm + lr have the same swizzle (wm and 32 i are
// multiples of 16), so row group i (or j) is the k-step's offset plus 4096 i bytes, an immediate of
// the LDS read: a stage's reads then cost one address add per k-step and operand.
struct FragOffsets {
  uint32_t a[kBK / 16], b[kBK / 16];
};
static_assert(FW_SWZ_SHIFT <= 2, "fragment offsets need rows r and r + 32 to share the swizzle");

template <int BM>
__device__ __forceinline__ FragOffsets frag_offsets(int wm, int wn, int lr, int lg) {
  FragOffsets o;
#pragma unroll
  for (int s = 0; s < kBK / 16; ++s) {
    o.a[s] = static_cast<uint32_t>(swz(wm + lr, 2 * s + lg) * 16);
    o.b[s] = static_cast<uint32_t>(BM * 128 + swz(wn + lr, 2 * s + lg) * 16);
  }
  return o;
}

template <int kTM, int kTN>
__device__ __forceinline__ void load_frags(const char* stage, const FragOffsets& o, Frags<kTM, kTN>& f) {
#pragma unroll
  for (int s = 0; s < kBK / 16; ++s) {
#pragma unroll
    for (int i = 0; i < kTM; ++i) f.a[s][i] = *reinterpret_cast<const h8v*>(stage + o.a[s] + 4096 * i);
#pragma unroll
    for (int j = 0; j < kTN; ++j) f.b[s][j] = *reinterpret_cast<const h8v*>(stage + o.b[s] + 4096 * j);
  }
}

// kT: accumulate the transposed tile (W rows as the MFMA A operand), so that acc[i][j][r] holds
// C[32 i + lane % 32][32 j + 8 (r / 4) + 4 g + r % 4]: four adjacent output columns per lane, which
// the epilogue then reads and writes as one 8-byte access.
template <int kTM, int kTN, bool kT>
__device__ __forceinline__ void mma_frags(const Frags<kTM, kTN>& f, f16v (&acc)[kTM][kTN]) {
#pragma unroll
  for (int s = 0; s < kBK / 16; ++s)
#pragma unroll
    for (int i = 0; i < kTM; ++i)
#pragma unroll
      for (int j = 0; j < kTN; ++j) {
        if constexpr (kT)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.b[s][j], f.a[s][i], acc[i][j], 0, 0, 0);
        else
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[s][i], f.b[s][j], acc[i][j], 0, 0, 0);
      }
}

// ---- direct-to-LDS pipeline (plain GEMMs) ------------------------------------------------------
// Per stage kt: wait until stage kt + 1 has landed, barrier (every wave also holds stage kt's operand
// fragments in registers by then, so its LDS slot is free), refill that slot with stage kt + ST,
// start the LDS reads of stage kt + 1's fragments, and run stage kt's MFMAs while they arrive. Copies
// have ST - 1 stages of MFMA time to land and LDS read latency is hidden behind the MFMAs.
// The LDS ring depth ST is picked per tile height: 256-row tiles use three 48 KB stages (one 8-wave
// block per CU); 128-row tiles (8 waves of 32 x 64; the split-k products) four 32 KB stages; 64-row
// tiles (launched when 128-row tiles would leave CUs idle) four 24 KB stages (5 or 6 measured the same).
// Tuning knobs (defaults measured on MI355X): ring depths per tile height, the minimum number of
// 256-row tiles for that shape, waves per 256-row and 64-row block, and the XCD rectangle grouping.
// 8 waves on the 64-row tiles (two per SIMD) against 4: out projection 14.8 -> 14.35 us, stem conv
// 36.0 -> 33.0 us (kernel trace, same box).
#ifndef FW_ST128
#define FW_ST128 4
#endif
#ifndef FW_ST64
#define FW_ST64 4
#endif
#ifndef FW_ST256
#define FW_ST256 3
#endif
#ifndef FW_ST192
#define FW_ST192 3
#endif
#ifndef FW_MIN_TILES256
#define FW_MIN_TILES256 128
#endif
template <int BM>
constexpr int dma_stages() {
  return BM == 256 ? FW_ST256 : BM == 192 ? FW_ST192 : BM == 128 ? FW_ST128 : FW_ST64;
}
// Ring depths: at least two stages (one read while the next lands) and a ring that fits the 160 KB of
// LDS of a CU; the vmcnt range of the explicit waits is checked where they are instantiated.
template <int BM>
constexpr bool ring_fits() { return dma_stages<BM>() >= 2 && dma_stages<BM>() * (BM + kBN) * 128 <= 160 * 1024; }
static_assert(ring_fits<256>() && ring_fits<192>() && ring_fits<128>() && ring_fits<64>(),
              "FW_ST256 / FW_ST192 / FW_ST128 / FW_ST64: 2 or more stages within 160 KB of LDS");
static_assert(FW_MIN_TILES256 >= 1, "FW_MIN_TILES256 must be positive");
// Waves per block, in gemm_wave_cols columns (kBN / cols output columns each) and waves / cols rows;
// each wave owns a (BM / rows) x (kBN / cols) tile. 192-row tiles use 2 x 4 waves of 96 x 32 and
// 128-row tiles 4 x 2 waves of 32 x 64.
#ifndef FW_W256
#define FW_W256 8
#endif
static_assert(FW_W256 == 2 || FW_W256 == 4 || FW_W256 == 8 || FW_W256 == 16,
              "FW_W256: 2 x (FW_W256 / 2) waves, each a whole number of 32-row MFMA tiles of the 256 rows");
#ifndef FW_W64
#define FW_W64 8  // waves per 64-row block: 8 (2 x 4 of 32 x 32) or 4 (2 x 2 of 32 x 64)
#endif
static_assert(FW_W64 == 4 || FW_W64 == 8, "FW_W64: 4 or 8 waves per 64-row block");
template <int BM>
constexpr int gemm_waves() { return BM == 256 ? FW_W256 : BM == 192 || BM == 128 ? 8 : FW_W64; }
template <int BM>
constexpr int gemm_wave_cols() { return BM == 192 || (BM == 64 && FW_W64 == 8) ? 4 : 2; }

// Source of the implicit conv's zero padding rows: a k stage of one A row is 64 halves.
__device__ __align__(16) _Float16 g_zero_row[kBK];

// CONV: implicit conv1d (k = 3, pad 1). A 64-wide k stage lies inside one tap (c_in % 64 == 0), so A
// row m of the stage is 64 contiguous channels of input row m * stride + tap - 1, or zeros outside
// [0, t_in).
template <int BM, bool CONV = false>
__device__ __forceinline__ void dma_stage(const GemmArgs& g, int m0, int n0, int k0, int wave, int lane,
                                          uint32_t lds_stage) {
  constexpr int kAInstr = BM / 8 / gemm_waves<BM>();  // wave instructions per A tile (8 rows each), per wave
  constexpr int kBInstr = kBN / 8 / gemm_waves<BM>();
  const int rsub = lane >> 3, slot = lane & 7;
  const int tap = CONV ? k0 / g.c_in : 0, ch0 = CONV ? k0 - tap * g.c_in : 0;
#pragma unroll
  for (int i = 0; i < kAInstr; ++i) {
    const int blk = wave * kAInstr + i;  // 8-row block of the tile
    const int row = blk * 8 + rsub;
    const int gm = min(m0 + row, g.m - 1);  // rows past m are computed and never stored
    const int chunk = swz_slot(row, slot);
    const _Float16* src;
    if constexpr (CONV) {
      const int r = gm * g.conv_stride + tap - 1;
      src = (r >= 0 && r < g.t_in) ? g.a + static_cast<size_t>(r) * g.c_in + ch0 + chunk * 8 : g_zero_row + chunk * 8;
    } else {
      src = g.a + static_cast<size_t>(gm) * g.lda + k0 + chunk * 8;
    }
    dma16(src, __builtin_amdgcn_readfirstlane(lds_stage + blk * 1024));
  }
#pragma unroll
  for (int i = 0; i < kBInstr; ++i) {
    const int blk = wave * kBInstr + i;
    const int row = blk * 8 + rsub;
    const int chunk = swz_slot(row, slot);
    dma16(g.w + static_cast<size_t>(n0 + row) * g.ldw + k0 + chunk * 8,
          __builtin_amdgcn_readfirstlane(lds_stage + BM * 128 + blk * 1024));
  }
}

// Plain GEMMs: the same copies with the k offset of a stage in the scalar base. Each lane keeps the
// byte offset of its 16-byte chunk (row * ld + swizzled chunk) for every copy it issues, so a stage
// costs kA + kB copy instructions and no vector address arithmetic (the per-stage 64-bit address
// updates were half the vector instructions of the main loop). The host keeps both operands below
// 4 GiB, the range of the 32-bit offsets.
template <int BM, int kNW>
struct CopyOffsets {
  static constexpr int kA = BM / 8 / kNW, kB = kBN / 8 / kNW;  // copies per wave and stage
  uint32_t a[kA], b[kB];
};

template <int BM, int kNW>
__device__ __forceinline__ void copy_offsets(const GemmArgs& g, int m0, int n0, int wave, int lane,
                                             CopyOffsets<BM, kNW>& c) {
  using C = CopyOffsets<BM, kNW>;
  const int rsub = lane >> 3, slot = lane & 7;
#pragma unroll
  for (int i = 0; i < C::kA; ++i) {
    const int row = (wave * C::kA + i) * 8 + rsub;
    const int gm = min(m0 + row, g.m - 1);  // rows past m are computed and never stored
    c.a[i] = static_cast<uint32_t>((static_cast<size_t>(gm) * g.lda + swz_slot(row, slot) * 8) * 2);
  }
#pragma unroll
  for (int i = 0; i < C::kB; ++i) {
    const int row = (wave * C::kB + i) * 8 + rsub;
    c.b[i] = static_cast<uint32_t>((static_cast<size_t>(n0 + row) * g.ldw + swz_slot(row, slot) * 8) * 2);
  }
}

template <int BM, int kNW>
__device__ __forceinline__ void dma_stage_s(const GemmArgs& g, const CopyOffsets<BM, kNW>& c, int kt, int wave,
                                            uint32_t lds_stage) {
  using C = CopyOffsets<BM, kNW>;
  const char* ab = reinterpret_cast<const char*>(g.a) + static_cast<size_t>(kt) * (kBK * 2);
  const char* wb = reinterpret_cast<const char*>(g.w) + static_cast<size_t>(kt) * (kBK * 2);
#pragma unroll
  for (int i = 0; i < C::kA; ++i) dma16_s(c.a[i], ab, lds_stage + (wave * C::kA + i) * 1024);
#pragma unroll
  for (int i = 0; i < C::kB; ++i) dma16_s(c.b[i], wb, lds_stage + BM * 128 + (wave * C::kB + i) * 1024);
}

// v columns of the q/k/v projection -> vt[head * 64 + d][vt_pos(t)]; rows in [m, vt_pad) get zeros so
// the padding keys of the last attention tile hold finite values. The tile is transposed through LDS
// (the operand ring is free once every wave has left the main loop): each lane puts its 4-row runs
// into a [128 columns][BM] staging tile, already in vt_pos order (tiles start at multiples of 64 and
// vt_pos permutes within 16-key groups), and the block then writes each column's BM keys as whole
// 16-byte chunks instead of one 8-byte store per 4 keys and column.
template <int BM, int kTM, int kTN>
__device__ __forceinline__ void store_vt(const GemmArgs& g, const f16v (&acc)[kTM][kTN], int m0, int n0, int wm,
                                         int wn, int lr, int lg, u32x4* lds) {
  constexpr int kStride = BM + 8;  // halves per staged column (16-byte aligned rows)
  static_assert(kBN * kStride * 2 <= dma_stages<BM>() * (BM + kBN) * 128, "staging tile must fit the ring");
  _Float16* t = reinterpret_cast<_Float16*>(lds);
  __syncthreads();  // every wave has read its last operand fragments from the ring
#pragma unroll
  for (int j = 0; j < kTN; ++j) {
    const int cl = wn + 32 * j + lr;
    const float b = g.bias ? h2f(g.bias[n0 + cl]) : 0.f;
#pragma unroll
    for (int i = 0; i < kTM; ++i)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int rl = wm + 32 * i + 8 * rq + 4 * lg;  // rows rl .. rl + 3 stay adjacent under vt_pos
        h4v v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = m0 + rl + e < g.m ? f2h(acc[i][j][4 * rq + e] + b) : static_cast<_Float16>(0.f);
        *reinterpret_cast<h4v*>(t + cl * kStride + vt_pos(rl)) = v;
      }
  }
  __syncthreads();
  constexpr int kChunks = BM / 8;  // 16-byte chunks per staged column
  _Float16* dst = g.vt + static_cast<size_t>(n0 - 2 * g.q_cols) * g.vt_pad;
  for (int c = threadIdx.x; c < kBN * kChunks; c += blockDim.x) {
    const int cl = c / kChunks, ch = c - cl * kChunks;
    const int pos = m0 + ch * 8;
    if (pos < g.vt_pad)
      *reinterpret_cast<u32x4*>(dst + static_cast<size_t>(cl) * g.vt_pad + pos) =
          *reinterpret_cast<const u32x4*>(t + cl * kStride + ch * 8);
  }
}

template <int BM, int EPI, bool CONV = false>
__global__ void __launch_bounds__(gemm_waves<BM>() * 64) gemm_dma_kernel(GemmArgs g) {
  constexpr int kDmaStages = dma_stages<BM>(), kNW = gemm_waves<BM>(), kNWN = gemm_wave_cols<BM>();
  constexpr int kWM = BM / (kNW / kNWN), kTM = kWM / 32, kTN = kBN / kNWN / 32;
  static_assert(kWM % 32 == 0 && kTN >= 1 && BM % (8 * kNW) == 0, "wave tiling");
  constexpr int kStageBytes = (BM + kBN) * 128;
  constexpr int kPerStage = (BM / 8 / kNW) + (kBN / 8 / kNW);  // copies per thread per stage
  // Transposed accumulators (8-byte epilogue accesses) pay off on the 64-row tiles of the 1280-column
  // GEMMs (fc2 44 -> 39 us, out projection 16 -> 13 us); on 256-row tiles they measured slower.
  constexpr bool kT = BM == 64 && EPI != kEpiQkvVt;
  __shared__ __align__(1024) u32x4 lds[kDmaStages * kStageBytes / 16];

  int m0, n0;
  tile_origin<BM>(g, m0, n0);
  int split = 0;
  if constexpr (EPI == kEpiPartial) {  // this block's k range: [split k, (split + 1) k) of the rows
    split = static_cast<int>(blockIdx.x) / ((g.n / kBN) * ((g.m + BM - 1) / BM));
    g.a += static_cast<size_t>(split) * g.k;
    g.w += static_cast<size_t>(split) * g.k;
  }
  // wave is uniform: the copies' LDS targets and the offsets that depend on it stay scalar
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave / kNWN) * kWM, wn = (wave % kNWN) * (kBN / kNWN);
  const int lr = lane & 31, lg = lane >> 5;
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
  const char* lds_bytes = reinterpret_cast<const char*>(lds);

  f16v acc[kTM][kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int j = 0; j < kTN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  CopyOffsets<BM, kNW> co;
  if constexpr (!CONV) copy_offsets<BM, kNW>(g, m0, n0, wave, lane, co);
  const FragOffsets fo = frag_offsets<BM>(wm, wn, lr, lg);
  auto issue = [&](int kt, int ring_slot) {  // stage kt's copies into ring slot ring_slot
    const uint32_t dst = lds0 + ring_slot * kStageBytes;
    if constexpr (CONV)
      dma_stage<BM, true>(g, m0, n0, kt * kBK, wave, lane, dst);
    else
      dma_stage_s<BM, kNW>(g, co, kt, wave, dst);
  };
  const int kt_n = g.k / kBK;
#pragma unroll
  for (int s = 0; s < kDmaStages; ++s)
    if (s < kt_n) issue(s, s);
  Frags<kTM, kTN> fa, fb;
  // this thread's copies of stage kt have landed once at most the later issued stages remain
  wait_stages_ahead<kPerStage, kDmaStages - 1>(min(kDmaStages - 1, kt_n - 1));
  barrier_only();
  load_frags<kTM, kTN>(lds_bytes, fo, fa);
  int cur = 0;  // ring slot of stage kt
  // stage kt with a stage kt + 1 after it
  auto step = [&](int kt, const Frags<kTM, kTN>& frags_kt, Frags<kTM, kTN>& nxt) {
    wait_stages_ahead<kPerStage, kDmaStages - 1>(min(kDmaStages - 2, kt_n - 2 - kt));
    lds_barrier();  // own fragment reads of stage kt done; stage kt + 1 visible; slot kt free
    if (kt + kDmaStages < kt_n) issue(kt + kDmaStages, cur);
    cur = cur + 1 == kDmaStages ? 0 : cur + 1;
    load_frags<kTM, kTN>(lds_bytes + cur * kStageBytes, fo, nxt);
    mma_frags<kTM, kTN, kT>(frags_kt, acc);
  };
  int kt = 0;
  for (; kt + 2 < kt_n; kt += 2) {
    step(kt, fa, fb);
    step(kt + 1, fb, fa);
  }
  if (kt + 1 < kt_n) {
    step(kt, fa, fb);
    mma_frags<kTM, kTN, kT>(fb, acc);
  } else {
    mma_frags<kTM, kTN, kT>(fa, acc);
  }

  if constexpr (kT) {
#pragma unroll
    for (int j = 0; j < kTN; ++j)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int col = n0 + wn + 32 * j + 8 * rq + 4 * lg;  // columns col .. col + 3
        h4v bb = {};
        if (g.bias) bb = *reinterpret_cast<const h4v*>(g.bias + col);
#pragma unroll
        for (int i = 0; i < kTM; ++i) {
          const int row = m0 + wm + 32 * i + lr;
          if (row < g.m) {
            h4v o;
            if constexpr (EPI == kEpiCrossKV) {
#pragma unroll
              for (int e = 0; e < 4; ++e) o[e] = f2h(acc[i][j][4 * rq + e] + h2f(bb[e]));
              const int d = col & 63, lhk = col >> 6;
              *reinterpret_cast<h4v*>(g.out + (static_cast<size_t>(lhk) * g.t_len + row) * 64 + d) = o;
            } else {
              h4v rv = {};
              if constexpr (epi_reads_res(EPI)) rv = *reinterpret_cast<const h4v*>(g.res + static_cast<size_t>(row) * g.ldr + col);
#pragma unroll
              for (int e = 0; e < 4; ++e)
                o[e] = f2h(epilogue_apply(EPI, acc[i][j][4 * rq + e], h2f(bb[e]), h2f(rv[e]), col + e, g.q_cols));
              *reinterpret_cast<h4v*>(g.out + static_cast<size_t>(row) * g.ldo + col) = o;
            }
          }
        }
      }
    return;
  }
  if constexpr (EPI == kEpiQkvVt) {
    if (n0 >= 2 * g.q_cols) {  // a v column tile (q_cols % 128 == 0): the branch is uniform per block
      store_vt<BM, kTM, kTN>(g, acc, m0, n0, wm, wn, lr, lg, lds);
      return;
    }
  }
#pragma unroll
  for (int j = 0; j < kTN; ++j) {
    const int col = n0 + wn + 32 * j + lr;
    const float b = g.bias ? h2f(g.bias[col]) : 0.f;
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * lg + (r & 3);
        if (row < g.m) {
          if constexpr (EPI == kEpiPartial) {
            g.part[(static_cast<size_t>(split) * g.m + row) * g.n + col] = acc[i][j][r];
          } else if constexpr (EPI == kEpiCrossKV) {
            const int d = col & 63, lhk = col >> 6;
            const size_t o = (static_cast<size_t>(lhk) * g.t_len + row) * 64 + d;
            g.out[o] = f2h(acc[i][j][r] + b);
          } else {
            g.out[static_cast<size_t>(row) * g.ldo + col] = f2h(epilogue_value(EPI, acc[i][j][r], b, g, row, col));
          }
        }
      }
    }
  }
}

template <int BM, int EPI, bool CONV>
__global__ void __launch_bounds__(256) gemm_kernel(GemmArgs g) {
  constexpr int kWM = BM / 2;                // wave tile rows
  constexpr int kTM = kWM / 32;              // MFMA tiles per wave along M
  constexpr int kTN = 2;                     // MFMA tiles per wave along N (64 columns)
  __shared__ __align__(16) u32x4 As0[BM * 8], As1[BM * 8];
  __shared__ __align__(16) u32x4 Bs0[kBN * 8], Bs1[kBN * 8];

  int m0, n0;
  tile_origin<BM>(g, m0, n0);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = (wave >> 1) * kWM, wn = (wave & 1) * 64;
  const int lr = lane & 31, lg = lane >> 5;

  f16v acc[kTM][kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int j = 0; j < kTN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  GemmStage<BM> st0, st1;
  const int kt_n = g.k / kBK;
  gemm_load<BM, CONV>(g, m0, n0, 0, tid, st0);
  gemm_store<BM>(As0, Bs0, tid, st0);
  if (kt_n > 1) gemm_load<BM, CONV>(g, m0, n0, kBK, tid, st1);
  __syncthreads();
  for (int kt = 0; kt < kt_n; kt += 2) {
    // stage kt in LDS buffer 0; stage kt + 1 arriving in st1
    if (kt + 2 < kt_n) gemm_load<BM, CONV>(g, m0, n0, (kt + 2) * kBK, tid, st0);
    gemm_mma<kTM, kTN>(As0, Bs0, wm, wn, lr, lg, acc);
    if (kt + 1 < kt_n) gemm_store<BM>(As1, Bs1, tid, st1);
    lds_barrier();
    if (kt + 1 >= kt_n) break;
    // stage kt + 1 in LDS buffer 1; stage kt + 2 arriving in st0
    if (kt + 3 < kt_n) gemm_load<BM, CONV>(g, m0, n0, (kt + 3) * kBK, tid, st1);
    gemm_mma<kTM, kTN>(As1, Bs1, wm, wn, lr, lg, acc);
    if (kt + 2 < kt_n) gemm_store<BM>(As0, Bs0, tid, st0);
    lds_barrier();
  }

#pragma unroll
  for (int j = 0; j < kTN; ++j) {
    const int col = n0 + wn + 32 * j + lr;
    const float b = g.bias ? h2f(g.bias[col]) : 0.f;
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * lg + (r & 3);
        if (row < g.m) {
          if constexpr (EPI == kEpiCrossKV) {
            // col = ((layer * 2 + kv) * heads + head) * 64 + d
            const int d = col & 63, lhk = col >> 6;
            const size_t o = (static_cast<size_t>(lhk) * g.t_len + row) * 64 + d;
            g.out[o] = f2h(acc[i][j][r] + b);
          } else {
            g.out[static_cast<size_t>(row) * g.ldo + col] = f2h(epilogue_value(EPI, acc[i][j][r], b, g, row, col));
          }
        }
      }
    }
  }
}

#ifndef FW_XCD_GROUP
#define FW_XCD_GROUP 1
#endif
static_assert(FW_XCD_GROUP == 0 || FW_XCD_GROUP == 1, "FW_XCD_GROUP is a switch (0 or 1)");
// Picks the XCD rectangle grid that divides the tile grid and moves the fewest bytes into the L2s:
// A is fetched once per column group (xn), W once per row group (xm).
void choose_xcd_groups(GemmArgs& g, int bm) {
  g.xm = g.xn = 0;
  if (!FW_XCD_GROUP || g.conv_stride) return;
  const int ntm = (g.m + bm - 1) / bm, ntn = g.n / kBN;
  double best = 0;
  for (int xm = 1; xm <= 8; xm *= 2) {
    const int xn = 8 / xm;
    if (ntm % xm || ntn % xn) continue;
    const double bytes = static_cast<double>(xn) * g.m * g.k + static_cast<double>(xm) * g.n * g.k;
    if (!g.xm || bytes < best) {
      best = bytes;
      g.xm = xm;
      g.xn = xn;
    }
  }
}

// The plain GEMMs address each operand as a scalar base plus a 32-bit per-lane byte offset
// (dma_stage_s): the rows a block reads must lie within 4 GiB of the operand's start.
bool copy_offsets_fit(const GemmArgs& g) {
  constexpr size_t kLimit = static_cast<size_t>(1) << 32;
  return (static_cast<size_t>(g.m - 1) * g.lda + kBK) * 2 < kLimit &&
         (static_cast<size_t>(g.n - 1) * g.ldw + kBK) * 2 < kLimit;
}

template <int BM>
int launch_gemm_bm(GemmArgs g, int epi, hipStream_t s) {
  const int tiles = (g.n / kBN) * ((g.m + BM - 1) / BM);
  const dim3 grid(tiles);
  choose_xcd_groups(g, BM);
  // Implicit convs with a long k (the stride-2 1280 -> 1280 stem conv, k = 3840) use the direct-to-LDS
  // pipeline (75 -> 37 us); with a short k (the 128 -> 1280 conv, k = 384: six stages) the ring's
  // fill and drain dominate and the register-staged kernel, whose small LDS footprint keeps two
  // blocks per CU, is faster (15 us against 18-19 us).
  if (g.conv_stride && g.k >= 1024) {
    switch (epi) {
#define FW_CONV_CASE(E) \
  case E:               \
    hipLaunchKernelGGL((gemm_dma_kernel<BM, E, true>), grid, dim3(gemm_waves<BM>() * 64), 0, s, g); break;
      FW_CONV_CASE(FW_EPI_BIAS)
      FW_CONV_CASE(FW_EPI_BIAS_GELU)
      FW_CONV_CASE(FW_EPI_BIAS_GELU_POS)
#undef FW_CONV_CASE
      default:
        return fw_fail(FW_EINVAL, "conv1d: unsupported epilogue %d", epi);
    }
    return fw_check_launch("conv1d");
  }
  if constexpr (BM <= 128) {
  if (g.conv_stride) {
    switch (epi) {
      case FW_EPI_BIAS: hipLaunchKernelGGL((gemm_kernel<BM, FW_EPI_BIAS, true>), grid, dim3(256), 0, s, g); break;
      case FW_EPI_BIAS_GELU:
        hipLaunchKernelGGL((gemm_kernel<BM, FW_EPI_BIAS_GELU, true>), grid, dim3(256), 0, s, g);
        break;
      case FW_EPI_BIAS_GELU_POS:
        hipLaunchKernelGGL((gemm_kernel<BM, FW_EPI_BIAS_GELU_POS, true>), grid, dim3(256), 0, s, g);
        break;
      default:
        return fw_fail(FW_EINVAL, "conv1d: unsupported epilogue %d", epi);
    }
    return fw_check_launch("conv1d");
  }
  }
  if (!copy_offsets_fit(g)) return fw_fail(FW_EINVAL, "gemm: each operand must span less than 4 GiB");
  switch (epi) {
#define FW_GEMM_CASE(E) \
  case E:               \
    hipLaunchKernelGGL((gemm_dma_kernel<BM, E>), grid, dim3(gemm_waves<BM>() * 64), 0, s, g); break;
    FW_GEMM_CASE(FW_EPI_BIAS)
    FW_GEMM_CASE(FW_EPI_BIAS_GELU)
    FW_GEMM_CASE(FW_EPI_BIAS_RESID)
    FW_GEMM_CASE(FW_EPI_BIAS_RESID_CLAMP)
    FW_GEMM_CASE(FW_EPI_BIAS_GELU_POS)
    FW_GEMM_CASE(FW_EPI_SCALE_Q)
    FW_GEMM_CASE(kEpiCrossKV)
    FW_GEMM_CASE(kEpiQkvVt)
#undef FW_GEMM_CASE
    default:
      return fw_fail(FW_EINVAL, "gemm: unknown epilogue %d", epi);
  }
  return fw_check_launch("gemm");
}

// 256-row tiles (8 waves, 48 KB stages) when they still cover half the CUs: they do twice the MFMA
// work per byte staged of 128-row tiles. When 256-row tiles would leave a quarter of the CUs idle and
// 192-row tiles still fit in one pass (q/k/v: 180 -> 240 tiles), 192-row tiles: each SIMD then does
// 3/4 of the MFMA work and each CU stages 5/6 of the bytes (4.90 -> 4.78 ms per encoder on MI355X).
// Fewer 128-row tiles than CUs leaves the chip idle: use 64-row tiles then. The implicit-GEMM conv
// stays on the register-staged kernel (<= 128 rows).
#ifndef FW_USE192
#define FW_USE192 1
#endif
static_assert(FW_USE192 == 0 || FW_USE192 == 1, "FW_USE192 is a switch (0 or 1)");
int launch_gemm(const GemmArgs& g, int epi, hipStream_t s) {
  const int tiles256 = (g.n / kBN) * ((g.m + 255) / 256);
  const int tiles192 = (g.n / kBN) * ((g.m + 191) / 192);
  const int tiles128 = (g.n / kBN) * ((g.m + 127) / 128);
  if (FW_USE192 && !g.conv_stride && tiles256 < 192 && tiles256 >= FW_MIN_TILES256 && tiles192 <= 256)
    return launch_gemm_bm<192>(g, epi, s);
  if (!g.conv_stride && tiles256 >= FW_MIN_TILES256) return launch_gemm_bm<256>(g, epi, s);
  if (tiles128 < 256) return launch_gemm_bm<64>(g, epi, s);
  return launch_gemm_bm<128>(g, epi, s);
}

// ------------------------------------------------------------------------------------------
// Row LayerNorm over 1280 columns: 32 lanes per row (5 x 16-byte chunks each), kLnRows = kLnThreads / 32 rows per block.
// ------------------------------------------------------------------------------------------
constexpr int kLnC = kHidden / 8 / 32;  // 16-byte fp16 chunks per lane of a row
#ifndef FW_LN_THREADS
#define FW_LN_THREADS 256
#endif
constexpr int kLnThreads = FW_LN_THREADS;  // threads per row-LayerNorm block: 32 lanes per row
constexpr int kLnRows = kLnThreads / 32;
static_assert(kLnThreads % 64 == 0 && kLnThreads <= 256, "whole waves, within the launch bounds");

// LayerNorm of one row held as v[] (this lane's elements: chunks sub + 32 c) with gamma / beta chunks
// gu / bu, written to yr when valid.
__device__ __forceinline__ void ln_row_finish(const float (&v)[kLnC * 8], const uint4 (&gu)[kLnC],
                                              const uint4 (&bu)[kLnC], float eps, uint4* yr, bool valid, int sub) {
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < kLnC * 8; ++i) sum += v[i];
  const float mean = group_sum<32>(sum) * (1.0f / kHidden);
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < kLnC * 8; ++i) {
    const float d = v[i] - mean;
    sq += d * d;
  }
  const float inv = rsqrtf(group_sum<32>(sq) * (1.0f / kHidden) + eps);
#pragma unroll
  for (int c = 0; c < kLnC; ++c) {
    const _Float16* gp = reinterpret_cast<const _Float16*>(&gu[c]);
    const _Float16* bp = reinterpret_cast<const _Float16*>(&bu[c]);
    uint4 o;
    _Float16* op = reinterpret_cast<_Float16*>(&o);
#pragma unroll
    for (int e = 0; e < 8; ++e) op[e] = f2h((v[c * 8 + e] - mean) * inv * h2f(gp[e]) + h2f(bp[e]));
    // computed outside the store's lane mask, so the gamma / beta requests are not sunk into it
    asm volatile("" : "+v"(o.x), "+v"(o.y), "+v"(o.z), "+v"(o.w));
    if (valid) yr[sub + 32 * c] = o;
  }
}

__global__ void __launch_bounds__(256) layernorm_rows_kernel(const _Float16* __restrict__ x,
                                                             const _Float16* __restrict__ gamma,
                                                             const _Float16* __restrict__ beta,
                                                             _Float16* __restrict__ y, int rows, float eps) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane & 31;
  const int row = blockIdx.x * kLnRows + wave * 2 + (lane >> 5);
  const bool valid = row < rows;
  const uint4* xr = reinterpret_cast<const uint4*>(x + static_cast<size_t>(valid ? row : 0) * kHidden);
  // gamma and beta are requested with the row, not after the two reductions
  const uint4* g4 = reinterpret_cast<const uint4*>(gamma);
  const uint4* b4 = reinterpret_cast<const uint4*>(beta);
  uint4 xu[kLnC], gu[kLnC], bu[kLnC];
#pragma unroll
  for (int c = 0; c < kLnC; ++c) xu[c] = xr[sub + 32 * c];
#pragma unroll
  for (int c = 0; c < kLnC; ++c) {
    gu[c] = g4[sub + 32 * c];
    bu[c] = b4[sub + 32 * c];
  }
  float v[kLnC * 8];
#pragma unroll
  for (int c = 0; c < kLnC; ++c) {
    const _Float16* hp = reinterpret_cast<const _Float16*>(&xu[c]);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[c * 8 + e] = h2f(hp[e]);
  }
  ln_row_finish(v, gu, bu, eps, reinterpret_cast<uint4*>(y + static_cast<size_t>(valid ? row : 0) * kHidden), valid,
                sub);
}

// The end of a split-k product followed by a LayerNorm: the split sums part[0 .. 1] of row r are added
// (in split order), then the residual epilogue of fw_gemm (FW_EPI_BIAS_RESID, or with CLAMP
// FW_EPI_BIAS_RESID_CLAMP) updates h[r] in place, and y[r] <- LN(h[r]) exactly as layernorm_rows_kernel.
template <bool CLAMP>
__global__ void __launch_bounds__(256) residual_layernorm_rows_kernel(const float* __restrict__ part,
                                                                      const _Float16* __restrict__ bias,
                                                                      _Float16* h,
                                                                      const _Float16* __restrict__ gamma,
                                                                      const _Float16* __restrict__ beta,
                                                                      _Float16* __restrict__ y, int rows, float eps) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane & 31;
  const int row = blockIdx.x * kLnRows + wave * 2 + (lane >> 5);
  const bool valid = row < rows;
  const size_t r0 = static_cast<size_t>(valid ? row : 0) * kHidden;
  const size_t split_stride = static_cast<size_t>(rows) * kHidden;
  const float4* p0 = reinterpret_cast<const float4*>(part + r0);
  const float4* p1 = reinterpret_cast<const float4*>(part + split_stride + r0);
  uint4* hr = reinterpret_cast<uint4*>(h + r0);
  const uint4* g4 = reinterpret_cast<const uint4*>(gamma);
  const uint4* b4 = reinterpret_cast<const uint4*>(beta);
  const uint4* bi4 = reinterpret_cast<const uint4*>(bias);
  uint4 hu[kLnC], gu[kLnC], bu[kLnC], biu[kLnC];
  float4 a0[kLnC][2], a1[kLnC][2];
#pragma unroll
  for (int c = 0; c < kLnC; ++c) {
    const int q = sub + 32 * c;  // this lane's 8-element chunk
    a0[c][0] = p0[2 * q];
    a0[c][1] = p0[2 * q + 1];
    a1[c][0] = p1[2 * q];
    a1[c][1] = p1[2 * q + 1];
    hu[c] = hr[q];
  }
#pragma unroll
  for (int c = 0; c < kLnC; ++c) {
    gu[c] = g4[sub + 32 * c];
    bu[c] = b4[sub + 32 * c];
    biu[c] = bi4[sub + 32 * c];
  }
  float v[kLnC * 8];
#pragma unroll
  for (int c = 0; c < kLnC; ++c) {
    const _Float16* rp = reinterpret_cast<const _Float16*>(&hu[c]);
    const _Float16* bp = reinterpret_cast<const _Float16*>(&biu[c]);
    const float* s0 = reinterpret_cast<const float*>(&a0[c][0]);
    const float* s1 = reinterpret_cast<const float*>(&a1[c][0]);
    uint4 o;
    _Float16* op = reinterpret_cast<_Float16*>(&o);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float acc = s0[e] + s1[e];
      float t = round_h(acc + h2f(bp[e]));
      if constexpr (CLAMP) {
        t = round_h(h2f(rp[e]) + t);
        const float lim = 65504.0f - 1000.0f;
        // the LayerNorm below reads the stored fp16 value: the bound itself rounds to 64512
        t = round_h(fminf(fmaxf(t, -lim), lim));
      } else {
        t = round_h(h2f(rp[e]) + t);
      }
      op[e] = f2h(t);
      v[c * 8 + e] = t;
    }
    asm volatile("" : "+v"(o.x), "+v"(o.y), "+v"(o.z), "+v"(o.w));
    if (valid) hr[sub + 32 * c] = o;
  }
  ln_row_finish(v, gu, bu, eps, reinterpret_cast<uint4*>(y + r0), valid, sub);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

}  // namespace
}  // namespace fw

using namespace fw;

extern "C" int fw_gemm(const void* a, int lda, const void* w, int ldw, const void* bias, void* out, int ldo,
                       const void* res, int ldr, int m, int n, int k, int epilogue, int q_cols, hipStream_t stream) {
  if (!a || !w || !out) return fw_fail(FW_EINVAL, "gemm: null pointer");
  if (m <= 0 || n <= 0 || k <= 0 || n % kBN || k % kBK)
    return fw_fail(FW_EINVAL, "gemm: need m > 0, n %% %d == 0, k %% %d == 0 (m=%d n=%d k=%d)", kBN, kBK, m, n, k);
  if (lda < k || ldw < k || ldo < n || lda % 8 || ldw % 8 || ldo % 8 || !aligned16(a) || !aligned16(w))
    return fw_fail(FW_EINVAL, "gemm: leading dimensions must cover the matrix and be multiples of 8");
  const bool needs_res = epilogue == FW_EPI_BIAS_RESID || epilogue == FW_EPI_BIAS_RESID_CLAMP ||
                         epilogue == FW_EPI_BIAS_GELU_POS;
  if (needs_res && (!res || ldr < n)) return fw_fail(FW_EINVAL, "gemm: epilogue %d needs res with ldr >= n", epilogue);
  if (!aligned8(out) || (bias && !aligned8(bias)) || (needs_res && (!aligned8(res) || ldr % 8)))
    return fw_fail(FW_EINVAL, "gemm: out, bias and res must be 8-byte aligned (and ldr a multiple of 8)");
  if (epilogue < FW_EPI_BIAS || epilogue > FW_EPI_SCALE_Q) return fw_fail(FW_EINVAL, "gemm: unknown epilogue %d", epilogue);
  GemmArgs g{static_cast<const _Float16*>(a), lda, static_cast<const _Float16*>(w), ldw,
             static_cast<const _Float16*>(bias), static_cast<_Float16*>(out), ldo,
             static_cast<const _Float16*>(res), ldr, m, n, k, q_cols, 0, 0, 0, 0, 0};
  return launch_gemm(g, epilogue, stream);
}

extern "C" int fw_conv1d(const void* x, int t_in, int c_in, int stride, const void* wp, const void* bias, void* out,
                         int c_out, const void* res, int epilogue, hipStream_t stream) {
  if (!x || !wp || !out) return fw_fail(FW_EINVAL, "conv1d: null pointer");
  if (t_in <= 0 || c_in <= 0 || c_in % 64 || c_out % kBN || (stride != 1 && stride != 2))
    return fw_fail(FW_EINVAL, "conv1d: need c_in %% 64 == 0, c_out %% %d == 0, stride 1 or 2", kBN);
  if (epilogue != FW_EPI_BIAS_GELU && epilogue != FW_EPI_BIAS_GELU_POS && epilogue != FW_EPI_BIAS)
    return fw_fail(FW_EINVAL, "conv1d: unsupported epilogue %d", epilogue);
  if (epilogue == FW_EPI_BIAS_GELU_POS && !res) return fw_fail(FW_EINVAL, "conv1d: positions required");
  if (!aligned16(x) || !aligned16(wp)) return fw_fail(FW_EINVAL, "conv1d: x and wp must be 16-byte aligned");
  const int t_out = (t_in - 1) / stride + 1;
  GemmArgs g{static_cast<const _Float16*>(x), c_in, static_cast<const _Float16*>(wp), 3 * c_in,
             static_cast<const _Float16*>(bias), static_cast<_Float16*>(out), c_out,
             static_cast<const _Float16*>(res), c_out, t_out, c_out, 3 * c_in, 0, stride, t_in, c_in, 0, 0};
  return launch_gemm(g, epilogue, stream);
}

extern "C" int fw_layernorm_rows(const void* x, const void* gamma, const void* beta, void* y, int rows, int n,
                                 float eps, hipStream_t stream) {
  if (!x || !gamma || !beta || !y) return fw_fail(FW_EINVAL, "layernorm_rows: null pointer");
  if (n != kHidden || rows <= 0) return fw_fail(FW_EINVAL, "layernorm_rows: n must be %d", kHidden);
  if (!aligned16(x) || !aligned16(y) || !aligned16(gamma) || !aligned16(beta))
    return fw_fail(FW_EINVAL, "layernorm_rows: tensors must be 16-byte aligned");
  hipLaunchKernelGGL(layernorm_rows_kernel, dim3((rows + kLnRows - 1) / kLnRows), dim3(kLnThreads), 0, stream,
                     static_cast<const _Float16*>(x), static_cast<const _Float16*>(gamma),
                     static_cast<const _Float16*>(beta), static_cast<_Float16*>(y), rows, eps);
  return fw_check_launch("layernorm_rows");
}

extern "C" int fw_gemm_splitk(const void* a, int lda, const void* w, int ldw, float* part, int m, int n, int k,
                              int splits, hipStream_t stream) {
  if (!a || !w || !part) return fw_fail(FW_EINVAL, "gemm_splitk: null pointer");
  if (splits != 2) return fw_fail(FW_EINVAL, "gemm_splitk: splits must be 2");
  if (m <= 0 || n <= 0 || n % kBN || k <= 0 || k % (splits * kBK))
    return fw_fail(FW_EINVAL, "gemm_splitk: need m > 0, n %% %d == 0, k %% %d == 0 (m=%d n=%d k=%d)", kBN,
                   splits * kBK, m, n, k);
  if (lda < k || ldw < k || lda % 8 || ldw % 8 || !aligned16(a) || !aligned16(w) || !aligned16(part))
    return fw_fail(FW_EINVAL, "gemm_splitk: leading dimensions must cover k and be multiples of 8; 16-byte aligned");
  GemmArgs g{};
  g.a = static_cast<const _Float16*>(a);
  g.lda = lda;
  g.w = static_cast<const _Float16*>(w);
  g.ldw = ldw;
  g.m = m;
  g.n = n;
  g.k = k / splits;  // per split
  g.splits = splits;
  g.part = part;
  // the XCD rectangles of the plain GEMMs (both k halves of a tile land on the same XCD when the tile
  // count is a multiple of 8): 126 -> 84 MB fetched from beyond L2 for the encoder's fc2
  choose_xcd_groups(g, 128);
  if (!copy_offsets_fit(g)) return fw_fail(FW_EINVAL, "gemm_splitk: each operand must span less than 4 GiB");
  const int tiles = (n / kBN) * ((m + 127) / 128);
  hipLaunchKernelGGL((gemm_dma_kernel<128, kEpiPartial>), dim3(splits * tiles), dim3(gemm_waves<128>() * 64), 0,
                     stream, g);
  return fw_check_launch("gemm_splitk");
}

extern "C" int fw_layernorm_rows_residual(const float* part, int splits, const void* bias, void* h,
                                          const void* gamma, const void* beta, void* y, int rows, int n, float eps,
                                          int epilogue, hipStream_t stream) {
  if (!part || !bias || !h || !gamma || !beta || !y) return fw_fail(FW_EINVAL, "layernorm_rows_residual: null pointer");
  if (splits != 2) return fw_fail(FW_EINVAL, "layernorm_rows_residual: splits must be 2");
  if (n != kHidden || rows <= 0) return fw_fail(FW_EINVAL, "layernorm_rows_residual: n must be %d", kHidden);
  if (epilogue != FW_EPI_BIAS_RESID && epilogue != FW_EPI_BIAS_RESID_CLAMP)
    return fw_fail(FW_EINVAL, "layernorm_rows_residual: epilogue must be a residual epilogue");
  if (!aligned16(part) || !aligned16(bias) || !aligned16(h) || !aligned16(gamma) || !aligned16(beta) || !aligned16(y))
    return fw_fail(FW_EINVAL, "layernorm_rows_residual: tensors must be 16-byte aligned");
  const dim3 grid((rows + kLnRows - 1) / kLnRows);
  if (epilogue == FW_EPI_BIAS_RESID_CLAMP)
    hipLaunchKernelGGL(residual_layernorm_rows_kernel<true>, grid, dim3(kLnThreads), 0, stream, part,
                       static_cast<const _Float16*>(bias), static_cast<_Float16*>(h),
                       static_cast<const _Float16*>(gamma), static_cast<const _Float16*>(beta),
                       static_cast<_Float16*>(y), rows, eps);
  else
    hipLaunchKernelGGL(residual_layernorm_rows_kernel<false>, grid, dim3(kLnThreads), 0, stream, part,
                       static_cast<const _Float16*>(bias), static_cast<_Float16*>(h),
                       static_cast<const _Float16*>(gamma), static_cast<const _Float16*>(beta),
                       static_cast<_Float16*>(y), rows, eps);
  return fw_check_launch("layernorm_rows_residual");
}


extern "C" int fw_encoder_qkv(const void* y, const void* w, const void* bias, void* qkv, void* vt, int seq, int heads,
                              hipStream_t stream) {
  if (!y || !w || !qkv || !vt) return fw_fail(FW_EINVAL, "encoder_qkv: null pointer");
  const int d = heads * kHeadDim;
  if (seq <= 0 || heads <= 0 || d % kBN || d % kBK)
    return fw_fail(FW_EINVAL, "encoder_qkv: need seq > 0 and heads * 64 a multiple of %d (seq=%d heads=%d)", kBN, seq,
                   heads);
  if (!aligned16(y) || !aligned16(w)) return fw_fail(FW_EINVAL, "encoder_qkv: y and w must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(vt) & 7u) return fw_fail(FW_EINVAL, "encoder_qkv: vt must be 8-byte aligned");
  GemmArgs g{static_cast<const _Float16*>(y), d, static_cast<const _Float16*>(w), d,
             static_cast<const _Float16*>(bias), static_cast<_Float16*>(qkv), 3 * d, nullptr, 0, seq, 3 * d, d, d,
             0, 0, 0, heads, seq, static_cast<_Float16*>(vt), vt_pad(seq)};
  return launch_gemm(g, kEpiQkvVt, stream);
}



extern "C" int fw_cross_kv(const void* enc, int t, const void* w, const void* bias, void* cross_kv, int layers,
                           int heads, hipStream_t stream) {
  if (!enc || !w || !cross_kv) return fw_fail(FW_EINVAL, "cross_kv: null pointer");
  if (t <= 0 || layers <= 0 || heads * kHeadDim != kHidden)
    return fw_fail(FW_EINVAL, "cross_kv: need t > 0, layers > 0, heads * 64 == %d", kHidden);
  if (!aligned16(enc) || !aligned16(w) || !aligned8(cross_kv) || (bias && !aligned8(bias)))
    return fw_fail(FW_EINVAL, "cross_kv: enc and w must be 16-byte aligned, cross_kv and bias 8-byte aligned");
  const int n = layers * 2 * kHidden;
  GemmArgs g{static_cast<const _Float16*>(enc), kHidden, static_cast<const _Float16*>(w), kHidden,
             static_cast<const _Float16*>(bias), static_cast<_Float16*>(cross_kv), 0, nullptr, 0, t, n, kHidden, 0,
             0, 0, 0, heads, t};
  return launch_gemm(g, kEpiCrossKV, stream);
}
