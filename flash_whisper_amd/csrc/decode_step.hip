// The decoder layers of one token (reference custom/model.py:107-121) as one persistent launch.
//
// The 34-launch step pays a kernel boundary between every pair of dependent operations: the end of
// a kernel writes its XCD's L2 back, the next kernel is dispatched and its blocks read the vector the
// previous one wrote from the MALL. Here one block per CU runs every operation of every layer in
// turn, and each operation hands its output vector to the next with tagged stores instead: every
// 8-byte word carries 4 bytes of payload (two fp16, or one fp32) and a 4-byte tag, written with one
// agent-scope store and read with agent-scope loads that repeat until the tag is the launch's (the
// low-latency protocol of ring collectives). A word's payload and tag arrive together, so no fence,
// flag or barrier sits between producer and consumer; a consumer waits one store-to-load trip.
//
// Per layer the operations ("phases") are those of the 34-launch step, with its arithmetic:
//   1 residual + LN1 + q/k/v GEMV          5 cross-attention splits (256 keys)
//   2 self-attention splits (64 keys)      6 combine + cross-out GEMV
//   3 combine + out GEMV                   7 residual + LN3 + fc1 + GELU
//   4 residual + LN2 + cross-q GEMV        8 fc2 GEMV
// Each phase runs on a run of blocks that did not work in the previous phase, so its workers have
// requested their weight rows (or K/V rows) before its input arrives. The residual stream lives in
// every block's LDS; a block adds the vectors it missed, in order, before its next LayerNorm. Every
// row's dot, the LayerNorm reductions (512-thread blocks, as the LN+GEMV launches), the split
// attention (4-wave items) and the combine are the device functions of the separate launches, so the
// outputs are bit-identical to the 34-launch step.
//
// Every wait is bounded: past a time limit a block flags an error in the control words and carries
// on with what it has, so the launch always drains. All blocks must be resident at once: one block
// per CU, and nothing else running on the device while the step runs.
#include <algorithm>
#include <type_traits>

#include "decode_dev.h"

namespace fw {
namespace {

constexpr int kStepWaves = 8;
constexpr int kStepThreads = kStepWaves * kWave;  // the LN+GEMV launches' block size: same LN reduction order
constexpr int kStepHeads = 20;
constexpr int kStepFfn = 4 * kHidden;
constexpr int kSelfSplitKeys = 64, kCrossSplitKeys = 256;
constexpr int kStepMaxLayers = 8;
constexpr int kStepMaxSteps = 1024;  // tokens one launch may decode
constexpr int kStepMaxEos = 4;       // end-of-text ids a launch stops at
constexpr int kPromptLen = 4;        // positions of the prompt pass (vectors per phase)
constexpr int kPartWords = kHeadDim + 2;  // acc[64], m, l of one split
constexpr int kPartRegion = kStepHeads * kMaxCombineSplits * kPartWords;
// Tagged-word regions of one layer (8-byte words; a vector of fp16 takes one word per pair)
constexpr int kQkvWords = 3 * kHidden / 2, kVecWords = kHidden / 2, kFfnWords = kStepFfn / 2;
constexpr int kOffQkv = 0;
constexpr int kOffSelfVec = kOffQkv + kQkvWords;     // self-attention output (640 words)
constexpr int kOffAttnOut = kOffSelfVec + kVecWords;
constexpr int kOffCrossQ = kOffAttnOut + kVecWords;
constexpr int kOffCrossPart = kOffCrossQ + kVecWords;
constexpr int kOffCrossVec = kOffCrossPart + kPartRegion;  // cross-attention output (640 words)
constexpr int kOffCrossOut = kOffCrossVec + kVecWords;
constexpr int kOffFfn = kOffCrossOut + kVecWords;
constexpr int kOffMlpOut = kOffFfn + kFfnWords;
constexpr int kLayerWords = kOffMlpOut + kVecWords;
// Workspace: control words ([0] epoch, [1] arrivals, [2] error), one bit per 8 KB page of the hand-off
// area (the half of the chip the page is local to), the latencies fw_decoder_step_calibrate measures, and
// the hand-off area (16 KB aligned). The regions below are laid out in logical words; logical page k
// (1024 words) has two physical copies, pages 2k and 2k + 1 of the area (see ll_store / ll_wait).
constexpr int kCtlBytes = 256;
constexpr int kGroupBytes = 256;
constexpr int kPageWords = 1024;               // 8 KB pages: memory alternates between the two halves of
constexpr int kMaxPages = kGroupBytes * 8;     // the chip every 8 KB (logical pages: one bit each)
constexpr int kCalibBytes = 2 * kMaxPages * 4;  // fp32 latency per logical page, for two pairs of XCDs
#ifndef FW_HX_PER_HALF
#define FW_HX_PER_HALF 1  // copies of every hand-off page on each half (1, 2 or 4; XCDs share them in turn)
#endif
static_assert(FW_HX_PER_HALF == 1 || FW_HX_PER_HALF == 2 || FW_HX_PER_HALF == 4, "FW_HX_PER_HALF");
constexpr int kCopies = 2 * FW_HX_PER_HALF;    // physical pages per logical page, alternating halves
constexpr size_t kAreaAlign = static_cast<size_t>(kCopies) * kPageWords * 8;  // a group never crosses 2 MB
// Worker counts of the phases that need few blocks (pairs of rows / items are spread over them).
constexpr int kVecWorkers = 80;    // 640 row pairs: one pair per wave
constexpr int kCrossWorkers = 120;  // 20 heads x 6 splits of the cross attention, one item per block
static_assert(kStepHeads * kHeadDim == kHidden, "20 heads of 64");
static_assert(kStepThreads == 512, "the LayerNorm reduction order of the 8-wave LN+GEMV launches");

struct StepLayer {
  const _Float16 *ln1_g, *ln1_b, *qkv_w, *qkv_b, *out_w, *out_b;
  const _Float16 *ln2_g, *ln2_b, *cq_w, *cq_b, *co_w, *co_b;
  const _Float16 *ln3_g, *ln3_b, *fc1_w, *fc1_b, *fc2_w, *fc2_b;
  float eps1, eps2, eps3;
  _Float16 *self_k, *self_v;
  const _Float16 *cross_k, *cross_v;
};

struct StepHead {
  const _Float16* gamma;
  const _Float16* beta;
  float eps;
  const _Float16* w;
  const int8_t* wq;
  const float2* meta;
  const uint8_t* suppress;
  int64_t* tokens;
  _Float16* y_out;        // optional: the final LayerNorm output, written by block 0
  int64_t* host_tokens;   // optional: host memory that receives every token as it is decoded
  int n_eos;              // the launch ends after a step whose token is one of eos[0 .. n_eos)
  int64_t eos[kStepMaxEos];
};

struct StepArgs {
  StepLayer layer[kStepMaxLayers];
  int n_layers;
  int64_t* cur;
  int64_t* state;
  const _Float16* embed;
  const _Float16* pos_embed;
  int vocab, max_pos, enc_len;
  float scale;
  _Float16* h_out;  // residual stream before the last fc2 output is added
  _Float16* x_out;  // last fc2 output
  unsigned char* ws;
  long long spin_limit;  // wall-clock ticks (100 MHz) a wait may take before it flags an error
  int has_head;          // run the final LN + LM head + argmax + finalize as the last phase
  int n_steps;           // tokens decoded by the launch (1 without the LM head)
  const int64_t* prompt;  // the prompt pass: the tokens of the launch's kPromptLen positions
  int lm_res_rows;        // LM-head rows per block resident in the launch's dynamic LDS
  StepHead head;
};

// The token a step embeds and the state word that gives its position: read from memory by the first
// step of a launch, then from the words the previous step's finalizing block broadcast.
struct StepPos {
  int64_t tok, pos_raw;
};

struct Ll {
  unsigned* ctl;
  unsigned tag;
  long long limit;
  int xcc;  // the XCD this block runs on (XCDs 0-3: half 0, XCDs 4-7: half 1)
};

// The two halves of an MI355X (XCDs 0-3 and 4-7, one I/O die each) reach memory on their own die
// faster: a tagged word whose 8 KB page is local to both producer and consumer hands off in about
// 0.4 us, one on the other die's memory in about 0.6 us (one producer and consumer on different dies:
// 0.5 us either way). Memory alternates between the dies every 8 KB, so logical page k of the hand-off
// area is stored in kCopies consecutive physical pages, kCopies k .. kCopies k + kCopies - 1, every
// other one on each die; which die the first is on is measured once per workspace
// (fw_decoder_step_calibrate). Every hand-off word is written to all of them, and each block polls
// one on its own die (the XCDs of a half take its copies in turn): the consumers of a word split over
// the copies.
__shared__ unsigned hx_groups[kMaxPages / 32];  // bit k: the first physical page of logical page k is on half 1
__device__ __forceinline__ int xcc_id() {
  unsigned x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  return static_cast<int>(x & 7u);
}
__device__ __forceinline__ uint64_t* hx_area(const unsigned char* ws) {
  const uintptr_t p = reinterpret_cast<uintptr_t>(ws) + kCtlBytes + kGroupBytes + kCalibBytes;
  return reinterpret_cast<uint64_t*>((p + kAreaAlign - 1) & ~(kAreaAlign - 1));
}
__device__ __forceinline__ const uint64_t* step_area();  // the launch's hand-off area (defined below)
// Physical word of logical word p (a pointer into the logical layout based at the area) in the copy that
// XCD x polls: on x's half, the (x mod FW_HX_PER_HALF)-th of that half's pages of the group.
__device__ __forceinline__ const uint64_t* hx_copy(const uint64_t* p, int x) {
  const uint64_t* base = step_area();
  const size_t w = static_cast<size_t>(p - base);
  const unsigned k = static_cast<unsigned>(w / kPageWords);
  const unsigned half = static_cast<unsigned>(x) >> 2, slot = static_cast<unsigned>(x) % FW_HX_PER_HALF;
  const unsigned sel = ((hx_groups[k >> 5] >> (k & 31)) & 1u) ^ half;
  return base + (static_cast<size_t>(k) * kCopies + 2 * slot + sel) * kPageWords + (w % kPageWords);
}

__device__ __forceinline__ uint64_t ll_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Stores logical word p in every copy.
__device__ __forceinline__ void ll_store(uint64_t* p, unsigned tag, unsigned v) {
  uint64_t* base = const_cast<uint64_t*>(step_area());
  const size_t w = static_cast<size_t>(p - base);
  uint64_t* q = base + (w / kPageWords) * kCopies * kPageWords + (w % kPageWords);
  const uint64_t x = (static_cast<uint64_t>(tag) << 32) | v;
#pragma unroll
  for (int j = 0; j < kCopies; ++j)
    __hip_atomic_store(q + j * kPageWords, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Payloads of the words buf[idx[k]] (idx[k] < 0: not wanted) once each carries the launch's tag. All
// words are requested at once and only the missing ones again, FW_LL_SLEEP x 64 clocks after the last
// poll came back (a longer sleep, and two polls of a word in flight at once, each measured slower). With
// kPlain the first read goes through the L2 (blocks of one XCD that read the same words then share one
// fetch); a word that comes back stale (an old tag: the L2 may hold a line from before its last write)
// is polled again with agent-scope loads, which always reach the coherent copy. Bounded: a wait that
// outlives the time limit, or that sees another block's error flag, stops and returns what it read.
#ifndef FW_LL_SLEEP
#define FW_LL_SLEEP 1
#endif
static_assert(FW_LL_SLEEP >= 0 && FW_LL_SLEEP <= 127, "s_sleep takes 0..127");
template <int N, bool kPlain = false>
__device__ __forceinline__ void ll_wait(const uint64_t* buf, const int (&idx)[N], unsigned (&val)[N], const Ll& c) {
  uint64_t w[N];
  const uint64_t* src[N];
  const uint64_t want = static_cast<uint64_t>(c.tag) << 32;
#pragma unroll
  for (int k = 0; k < N; ++k) src[k] = hx_copy(buf + (idx[k] >= 0 ? idx[k] : 0), c.xcc);
#pragma unroll
  for (int k = 0; k < N; ++k) w[k] = idx[k] >= 0 ? (kPlain ? *src[k] : ll_load(src[k])) : want;
  static_assert(N <= 64, "one pending bit per word");
  unsigned long long pending = 0;
#pragma unroll
  for (int k = 0; k < N; ++k)
    pending |= static_cast<unsigned long long>(static_cast<unsigned>(w[k] >> 32) != c.tag) << k;
  if (pending) {
    const long long t0 = wall_clock64();
    for (int it = 1; pending; ++it) {
      if (!kPlain || it > 1) __builtin_amdgcn_s_sleep(FW_LL_SLEEP);
#pragma unroll
      for (int k = 0; k < N; ++k)
        if (pending >> k & 1ull) w[k] = ll_load(src[k]);
      pending = 0;
#pragma unroll
      for (int k = 0; k < N; ++k)
        pending |= static_cast<unsigned long long>(static_cast<unsigned>(w[k] >> 32) != c.tag) << k;
      if (pending && (it & 15) == 0) {
        if (__hip_atomic_load(c.ctl + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) break;
        if (wall_clock64() - t0 > c.limit) {
          __hip_atomic_store(c.ctl + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
      }
    }
  }
#pragma unroll
  for (int k = 0; k < N; ++k) val[k] = static_cast<unsigned>(w[k]);
}

__device__ __forceinline__ unsigned half_bits(_Float16 x) { return __builtin_bit_cast(unsigned short, x); }

// ---------------------------------------------------------------------------------------------
// Phase timeline (built only with FW_STEP_TIMELINE=1, a profiling build of the library): thread 0 of
// every block notes the 100 MHz wall clock at fixed points of each step in LDS (a global store would
// add its completion to the next wait on the vector-memory counter), and waves 1-2 copy the step's
// slots to a buffer set with fw_decoder_step_timeline once the step is done: slot s of block b in step
// st at [(st * G + b) * kTlSlots + s]. Slot 0 is the step's start, layer l < kTlLayers phase p (1..8)
// has slots tl_phase(l, p) + {0 entered and its loads issued, 1 input in (after the prologue), 2 output
// stored, 3 the cross attention's combine stored, the self attention's split rounds done, or a
// LayerNorm phase's residual contributions added (thread 0's share)}, the LM
// head the slots from kTlLm on (TlLm), layer 0's self attention a few more from kTlSa on (TlSa) and
// each of its waves' partials from kTlWave on. In the
// product build every mark is empty.
// ---------------------------------------------------------------------------------------------
#ifndef FW_STEP_TIMELINE
#define FW_STEP_TIMELINE 0
#endif
constexpr int kTlLayers = 4, kTlSlots = 160, kTlLm = 1 + kTlLayers * 8 * 4;
enum TlLm { kTlArrive = 0, kTlY, kTlDigits, kTlRegScored, kTlResScored, kTlScored, kTlCand, kTlMaxStored,
            kTlFinGathered, kTlFinStored, kTlCaught, kTlBatch0 };
constexpr int kTlSa = kTlLm + 12;
enum TlSa { kTlSaRow = 0, kTlSaPartial, kTlSaMerged, kTlSaBarrier };
static_assert(kTlSa + kTlSaBarrier < kTlSlots, "timeline slots");
// The shader clock (s_memtime) at the step's start and end and the wall clock at its end: their ratio
// to the wall clock gives the core clock the step ran at.
constexpr int kTlClk = kTlSa + 8;
enum TlClk { kTlClkStart = 0, kTlClkEnd, kTlClkWallEnd };
static_assert(kTlClk + kTlClkWallEnd < kTlSlots, "timeline slots");
// Layer 0's self attention: each wave's partials done (lane 0 of wave w marks slot kTlWave + w).
constexpr int kTlWave = kTlClk + 3;
static_assert(kTlWave + kStepWaves <= kTlSlots, "timeline slots");
__host__ __device__ constexpr int tl_phase(int l, int p) { return 1 + (l * 8 + (p - 1)) * 4; }
#if FW_STEP_TIMELINE
__device__ long long* g_step_tl;  // [steps][G][kTlSlots], or null
__device__ int g_step_tl_steps;   // steps the buffer holds
__shared__ long long tl_lds[kTlSlots];
#endif
struct Tl {
#if FW_STEP_TIMELINE
  long long* p;  // the step's slots of this block in the buffer, or null
  __device__ void mark(int s) const {
    if (p && threadIdx.x == 0) tl_lds[s] = wall_clock64();
  }
  __device__ void phase(int l, int ph, int k) const {
    if (l < kTlLayers) mark(tl_phase(l, ph) + k);
  }
  __device__ void mark_wave(int s) const {
    if (p && (threadIdx.x & (kWave - 1)) == 0) tl_lds[s + threadIdx.x / kWave] = wall_clock64();
  }
  __device__ void mark_shader_clock(int s) const {
    if (p && threadIdx.x == 0) tl_lds[s] = static_cast<long long>(__builtin_amdgcn_s_memtime());
  }
  // After a barrier that ends the step: waves 1-2 copy the slots out and clear them (wave 0 may be
  // polling the next step's words, and its loads would wait behind these stores).
  __device__ void flush() const {
    const int t = threadIdx.x - kWave;
    if (p && t >= 0 && t < kTlSlots) {
      p[t] = tl_lds[t];
      tl_lds[t] = 0;
    }
  }
  __device__ static Tl at(int st) {
    return {g_step_tl && st < g_step_tl_steps
                ? g_step_tl + (static_cast<size_t>(st) * gridDim.x + blockIdx.x) * kTlSlots
                : nullptr};
  }
  __device__ static void clear() {
    if (threadIdx.x < kTlSlots) tl_lds[threadIdx.x] = 0;
  }
#else
  __device__ void mark(int) const {}
  __device__ void phase(int, int, int) const {}
  __device__ void mark_wave(int) const {}
  __device__ void mark_shader_clock(int) const {}
  __device__ void flush() const {}
  __device__ static Tl at(int) { return {}; }
  __device__ static void clear() {}
#endif
};

// ---------------------------------------------------------------------------------------------
// GEMV rows. A wave owns row pairs: for K = 1280 rows 2q and 2q + 1 side by side (32 lanes each, as
// gemv_kernel), for K = 5120 one after the other (64 lanes each). Lane 0 stores the pair's word.
// Rows are requested by gv_load before the phase's input arrives and scored by gv_finish.
// ---------------------------------------------------------------------------------------------
constexpr int kMaxPasses = 3;  // row pairs per wave requested ahead (the U of Gv)

template <int K, int U>
struct Gv {
  static_assert(U >= 1 && U <= kMaxPasses, "the output staging holds kMaxPasses words per wave");
  using RS = RowSplit<K>;
  static constexpr int kRowsPerPair = K == kHidden ? 1 : 2;  // rows per pair held by one lane
  uint4 w[U][kRowsPerPair][RS::kC];
  _Float16 b[U][kRowsPerPair];
  int q[U];  // pair index, or -1
};

template <int K, int U>
__device__ __forceinline__ void gv_load(Gv<K, U>& g, const _Float16* __restrict__ w, const _Float16* __restrict__ bias,
                                        int npairs, int q0, int qstride) {
  using RS = RowSplit<K>;
  const int lane = threadIdx.x & 63, sub = lane % RS::kLPR, rsel = lane / RS::kLPR;
  const uint4* w4 = reinterpret_cast<const uint4*>(w);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int q = q0 + u * qstride;
    g.q[u] = q < npairs ? q : -1;
    const int qc = q < npairs ? q : npairs - 1;
#pragma unroll
    for (int r = 0; r < Gv<K, U>::kRowsPerPair; ++r) {
      const int row = K == kHidden ? 2 * qc + rsel : 2 * qc + r;
      g.b[u][r] = *(bias ? bias + row : &g_zero_half);
#pragma unroll
      for (int c = 0; c < RS::kC; ++c) g.w[u][r][c] = ld_weights(w4 + static_cast<size_t>(row) * RS::kChunksRow + sub + RS::kLPR * c);
    }
  }
}

// Scores the pairs requested by gv_load, then stores the block's words: wave w's word of pass u is
// word base + u * qs + w, so each pass gives a run of 8 consecutive words, staged in LDS and written by
// 8 lanes of wave 0 with one store (one coalesced write per line instead of one per wave). All waves
// of the block call it (it has a barrier).
template <int K, int U, int ACT>
__device__ __forceinline__ void gv_finish(const Gv<K, U>& g, const _Float16* x_lds, unsigned* stage, uint64_t* out,
                                          unsigned tag, _Float16* plain_out, int base, int qs, int npairs) {
  using RS = RowSplit<K>;
  const int lane = threadIdx.x & 63, sub = lane % RS::kLPR, wave = threadIdx.x >> 6;
  uint4 xr[RS::kC];
#pragma unroll
  for (int c = 0; c < RS::kC; ++c) xr[c] = reinterpret_cast<const uint4*>(x_lds)[sub + RS::kLPR * c];
  if constexpr (ACT == FW_ACT_GELU && K == kHidden && U > 1) {
    // The U row pairs' GELUs in one evaluation: after the row sums every lane of a 32-lane half holds its
    // row's value, so lanes 8u .. 8u + 7 of each half take pass u's and one erf covers all passes (the same
    // function of the same fp32 values as one evaluation per pass; erf is most of a pass's instructions).
    static_assert(U <= 4, "8 lanes per pass in each half");
    float z = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {  // passes past the rows (q < 0) score a clamped row; their values are dropped
      float acc = 0.f;
#pragma unroll
      for (int c = 0; c < RS::kC; ++c) acc = dot8(g.w[u][0][c], xr[c], acc);
      acc = group_sum<RS::kLPR>(acc);
      const float y = acc + h2f(g.b[u][0]);
      z = ((lane & 31) >> 3) == u ? y : z;
    }
    float gz = gelu_erf(round_h(z));
    asm volatile("" : "+v"(gz));  // rounded to fp32 first, as gemv_kernel does (see below)
    const int gb = static_cast<int>(half_bits(f2h(gz)));
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const unsigned lo = static_cast<unsigned>(__builtin_amdgcn_readlane(gb, 8 * u));
      const unsigned hi = static_cast<unsigned>(__builtin_amdgcn_readlane(gb, 32 + 8 * u));
      if (g.q[u] >= 0 && lane == 0) stage[u * kStepWaves + wave] = lo | (hi << 16);
    }
  } else {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (g.q[u] < 0) continue;  // wave-uniform
    unsigned bits[Gv<K, U>::kRowsPerPair];
#pragma unroll
    for (int r = 0; r < Gv<K, U>::kRowsPerPair; ++r) {
      float acc = 0.f;
#pragma unroll
      for (int c = 0; c < RS::kC; ++c) acc = dot8(g.w[u][r][c], xr[c], acc);
      acc = group_sum<RS::kLPR>(acc);
      float y = acc + h2f(g.b[u][r]);
      if constexpr (ACT == FW_ACT_GELU) y = gelu_erf(round_h(y));
      // y is rounded to fp32 first, as gemv_kernel does (its store pins y the same way): without the
      // pin the compiler may fold the GELU's last product into the fp16 conversion (one rounding
      // instead of two), which differs in rare elements
      asm volatile("" : "+v"(y));
      bits[r] = half_bits(f2h(y));
    }
    unsigned lo, hi;
    if constexpr (K == kHidden) {
      lo = bits[0];
      hi = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(bits[0]), 32));
    } else {
      lo = bits[0];
      hi = bits[1];
    }
    if (lane == 0) stage[u * kStepWaves + wave] = lo | (hi << 16);
  }
  }
  __syncthreads();
  if (threadIdx.x < U * kStepWaves) {
    const int u = threadIdx.x / kStepWaves, q = base + u * qs + threadIdx.x % kStepWaves;
    if (q < npairs) {
      const unsigned word = stage[threadIdx.x];
      ll_store(out + q, tag, word);
      if (plain_out) reinterpret_cast<unsigned*>(plain_out)[q] = word;
    }
  }
}

// gv_finish for NV input vectors (x_lds holds them K halves apart): the rows requested once are dotted
// with every vector, each with gemv_kernel's arithmetic; vector v's words go to out + v * npairs.
template <int K, int U, int ACT, int NV>
__device__ __forceinline__ void gv_finish_nv(const Gv<K, U>& g, const _Float16* x_lds, unsigned* stage, uint64_t* out,
                                             unsigned tag, int base, int qs, int npairs) {
  if constexpr (NV == 1) {
    gv_finish<K, U, ACT>(g, x_lds, stage, out, tag, nullptr, base, qs, npairs);
  } else {
    using RS = RowSplit<K>;
    const int lane = threadIdx.x & 63, sub = lane % RS::kLPR, wave = threadIdx.x >> 6;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      uint4 xr[RS::kC];
#pragma unroll
      for (int c = 0; c < RS::kC; ++c) xr[c] = reinterpret_cast<const uint4*>(x_lds + v * K)[sub + RS::kLPR * c];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (g.q[u] < 0) continue;  // wave-uniform
        unsigned bits[Gv<K, U>::kRowsPerPair];
#pragma unroll
        for (int r = 0; r < Gv<K, U>::kRowsPerPair; ++r) {
          float acc = 0.f;
#pragma unroll
          for (int c = 0; c < RS::kC; ++c) acc = dot8(g.w[u][r][c], xr[c], acc);
          acc = group_sum<RS::kLPR>(acc);
          float y = acc + h2f(g.b[u][r]);
          if constexpr (ACT == FW_ACT_GELU) y = gelu_erf(round_h(y));
          asm volatile("" : "+v"(y));  // rounded to fp32 first, as in gv_finish
          bits[r] = half_bits(f2h(y));
        }
        unsigned lo, hi;
        if constexpr (K == kHidden) {
          lo = bits[0];
          hi = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(bits[0]), 32));
        } else {
          lo = bits[0];
          hi = bits[1];
        }
        if (lane == 0) stage[(v * U + u) * kStepWaves + wave] = lo | (hi << 16);
      }
    }
    __syncthreads();
    if (threadIdx.x < NV * U * kStepWaves) {
      const int t = threadIdx.x, v = t / (U * kStepWaves), r = t % (U * kStepWaves);
      const int q = base + (r / kStepWaves) * qs + r % kStepWaves;
      if (q < npairs) ll_store(out + static_cast<size_t>(v) * npairs + q, tag, stage[t]);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// The residual stream is the token + position embedding plus, per layer, the out, cross-out and fc2
// outputs ("contributions" 0, then 1 + 3 l + {0, 1, 2}). A block keeps the count it has added; one
// that works in a LayerNorm phase first adds, in order, every contribution it has not.
// ---------------------------------------------------------------------------------------------
// With NV vectors per phase (the prompt pass) every region holds NV copies back to back.
template <int NV = 1>
__device__ __forceinline__ const uint64_t* contribution(uint64_t* regions, int i) {
  const int l = (i - 1) / 3, k = (i - 1) % 3;
  return regions + static_cast<size_t>(l) * NV * kLayerWords +
         NV * (k == 0 ? kOffAttnOut : (k == 1 ? kOffCrossOut : kOffMlpOut));
}

// Phases without a LayerNorm (out, cross-out, fc2) add the residual contributions published before
// their input while they wait for it (the same adds in the same order), so fewer are left for the
// block's next LayerNorm, and the blocks that ran the last fc2 reach the LM head with only that output
// to add.
#ifndef FW_EAGER_CATCH_UP
#define FW_EAGER_CATCH_UP 1
#endif
#ifndef FW_CATCH_GROUP
#define FW_CATCH_GROUP 1  // residual contributions awaited together by a 512-thread catch-up (4 measured 3.6 us a step slower)
#endif
static_assert(FW_CATCH_GROUP >= 1 && FW_CATCH_GROUP <= 8, "FW_CATCH_GROUP");
// Adds the contributions applied .. upto - 1 to h_res, in order; run by kThreads threads (the block, or
// one wave), t the thread's index among them. With NV vectors per phase, h_res holds NV residual
// streams and vectors V0 .. NV - 1 are brought up to date (vector v embeds prompt token v at position
// pos_raw + v). Up to kGroup pending contributions are awaited with one wait (one memory round trip for
// all of them), then added one after another.
template <int kThreads = kStepThreads, int NV = 1, int V0 = 0>
__device__ __forceinline__ void resid_catch_up(_Float16* h_res, int& applied, int upto, uint64_t* regions,
                                               const StepArgs& a, const Ll& c, const StepPos& sp,
                                               int t = threadIdx.x) {
  constexpr int kWords = (NV - V0) * kVecWords;  // the vectors' pairs, vector-major from V0
  constexpr int kPer = (kWords + kThreads - 1) / kThreads;
  constexpr int kGroup = kThreads >= kStepThreads && NV == 1 ? FW_CATCH_GROUP : 1;  // bounded by the registers it takes
  static_assert(kGroup * kPer <= 64, "one pending bit per word");
  h2v* h2 = reinterpret_cast<h2v*>(h_res) + V0 * kVecWords;
  while (applied < upto) {  // uniform over the threads
    if (applied == 0) {
      if constexpr (NV == 1) {
        const _Float16 *ea, *eb;
        embed_rows_of(sp.tok, sp.pos_raw, a.embed, a.pos_embed, a.vocab, a.max_pos, &ea, &eb);
        const h2v* a2 = reinterpret_cast<const h2v*>(ea);
        const h2v* b2 = reinterpret_cast<const h2v*>(eb);
        for (int i = t; i < kVecWords; i += kThreads) {
          const h2v p = a2[i], q = b2[i];
          h2v o;
          o.x = f2h(h2f(p.x) + h2f(q.x));
          o.y = f2h(h2f(p.y) + h2f(q.y));
          h2[i] = o;
        }
      } else {
        for (int w = t; w < kWords; w += kThreads) {
          const int v = V0 + w / kVecWords, i = w % kVecWords;
          const _Float16 *ea, *eb;
          embed_rows_of(a.prompt[v], sp.pos_raw + v, a.embed, a.pos_embed, a.vocab, a.max_pos, &ea, &eb);
          const h2v p = reinterpret_cast<const h2v*>(ea)[i], q = reinterpret_cast<const h2v*>(eb)[i];
          h2v o;
          o.x = f2h(h2f(p.x) + h2f(q.x));
          o.y = f2h(h2f(p.y) + h2f(q.y));
          h2[w] = o;
        }
      }
      ++applied;
    } else {
      const int ng = min(upto - applied, kGroup);  // contributions awaited together
      int idx[kGroup * kPer];
#pragma unroll
      for (int g = 0; g < kGroup; ++g) {
        const int off = g < ng ? static_cast<int>(contribution<NV>(regions, applied + g) - regions) + V0 * kVecWords : 0;
#pragma unroll
        for (int k = 0; k < kPer; ++k)
          idx[g * kPer + k] = g < ng && t + k * kThreads < kWords ? off + t + k * kThreads : -1;
      }
      unsigned v[kGroup * kPer];
      ll_wait<kGroup * kPer>(regions, idx, v, c);
      // the thread's pairs read first (one batch of LDS reads: a branch per pair made each read a round
      // trip of its own), the contributions added in order (every add rounds to fp16), then stored
      h2v hv[kPer];
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        const int w = t + k * kThreads;
        hv[k] = h2[w < kWords ? w : 0];
      }
#pragma unroll
      for (int g = 0; g < kGroup; ++g) {
        if (g >= ng) break;  // uniform
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
          const h2v xp = __builtin_bit_cast(h2v, v[g * kPer + k]);
          h2v o;
          o.x = f2h(h2f(hv[k].x) + h2f(xp.x));
          o.y = f2h(h2f(hv[k].y) + h2f(xp.y));
          hv[k] = o;
        }
      }
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        const int w = t + k * kThreads;
        if (w < kWords) h2[w] = hv[k];
      }
      applied += ng;
    }
  }
}

// Contribution 0 (the token + position embedding, resid_catch_up's first add) in two steps, so a phase can
// request the rows before its weight rows: the rows come back first (loads return in order) and the add
// does not wait for the weights.
struct EmbRegs {
  h2v p[2], q[2];
};
__device__ __forceinline__ void embed_load(EmbRegs& e, const StepArgs& a, const StepPos& sp) {
  const _Float16 *ea, *eb;
  embed_rows_of(sp.tok, sp.pos_raw, a.embed, a.pos_embed, a.vocab, a.max_pos, &ea, &eb);
  const int t = threadIdx.x;
  const int i1 = t + kStepThreads < kVecWords ? t + kStepThreads : t;  // threads past the pairs repeat theirs
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int i = k == 0 ? t : i1;
    e.p[k] = reinterpret_cast<const h2v*>(ea)[i];
    e.q[k] = reinterpret_cast<const h2v*>(eb)[i];
  }
}
__device__ __forceinline__ void embed_store(const EmbRegs& e, _Float16* h_res, int& applied) {
  h2v* h2 = reinterpret_cast<h2v*>(h_res);
  const int t = threadIdx.x;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int i = t + k * kStepThreads;
    if (i < kVecWords) {
      h2v o;
      o.x = f2h(h2f(e.p[k].x) + h2f(e.q[k].x));
      o.y = f2h(h2f(e.p[k].y) + h2f(e.q[k].y));
      h2[i] = o;
    }
  }
  applied = 1;
}

// y = LN(h_res) with gamma / beta, the arithmetic of ln_finish<512, true> on the (already rounded)
// residual: ln_params requests gamma and beta (before the phase's input is awaited), resid_layernorm
// takes the residual pairs each thread owns (the ones it wrote itself) and finishes the LayerNorm.
__device__ __forceinline__ void ln_params(LnRegs<kStepThreads>& in, const _Float16* gamma, const _Float16* beta) {
  const h2v* g2 = reinterpret_cast<const h2v*>(gamma);
  const h2v* be2 = reinterpret_cast<const h2v*>(beta);
  const h2v zero = {static_cast<_Float16>(0.f), static_cast<_Float16>(0.f)};
#pragma unroll
  for (int i = 0; i < LnRegs<kStepThreads>::kPer; ++i) {
    const int idx = threadIdx.x + i * kStepThreads;
    const bool ok = idx < LnRegs<kStepThreads>::kPairs;
    in.a[i] = in.b[i] = zero;
    in.g[i] = ok ? g2[idx] : zero;
    in.be[i] = ok ? be2[idx] : zero;
  }
}

__device__ __forceinline__ void resid_layernorm(LnRegs<kStepThreads>& in, const _Float16* h_res, float eps,
                                                _Float16* y, float* red) {
  const h2v* h2 = reinterpret_cast<const h2v*>(h_res);
#pragma unroll
  for (int i = 0; i < LnRegs<kStepThreads>::kPer; ++i) {
    const int idx = threadIdx.x + i * kStepThreads;
    if (idx < LnRegs<kStepThreads>::kPairs) in.a[i] = h2[idx];
  }
  ln_finish<kStepThreads, true>(in, false, nullptr, eps, y, red);
}

// resid_layernorm for NV residual streams (kHidden apart in h_res and y): the vectors share each
// reduction round (ln_finish_multi), each vector's result that of resid_layernorm on it alone.
template <int NV>
__device__ __forceinline__ void resid_layernorm_nv(LnRegs<kStepThreads>& lnr, const _Float16* h_res, float eps,
                                                   _Float16* y, float* red) {
  if constexpr (NV == 1) {
    resid_layernorm(lnr, h_res, eps, y, red);  // each thread reads the pairs it brought up to date itself
  } else {
    __syncthreads();  // the catch-up spread the NV vectors' pairs over the threads differently
    LnRegs<kStepThreads> in[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      in[v] = lnr;
      const h2v* h2 = reinterpret_cast<const h2v*>(h_res + v * kHidden);
#pragma unroll
      for (int i = 0; i < LnRegs<kStepThreads>::kPer; ++i) {
        const int idx = threadIdx.x + i * kStepThreads;
        if (idx < LnRegs<kStepThreads>::kPairs) in[v].a[i] = h2[idx];
      }
    }
    ln_finish_multi<kStepThreads, NV>(in, false, nullptr, eps, y, red);
  }
}

// ---------------------------------------------------------------------------------------------
// Split attention items: item i of a phase is (head i / nsplit, split i % nsplit); a block runs two
// at once, waves 0-3 and 4-7, each exactly as attn_split_kernel<MAXP, false, 4> runs one block.
// ---------------------------------------------------------------------------------------------
struct AttnLds {
  float wm[2][4], wl[2][4];
  float wacc[2][4][kHeadDim];
  uint4 q[2][3][8];  // q, fresh k, fresh v of the item's head (8 chunks of 8 fp16 each)
};

// Thread d < 64's element of one head's attention output from its split partials: get(s, m, l, a)
// gives split s's max, exp-sum and value sum for element d (s < ns; splits past ns are empty). The
// arithmetic is combine_finish's over kMaxCombineSplits slots: the maximum first, then per split in
// order the weight, the denominator's and the numerator's fused adds (the two sums independent, so one
// pass keeps each in split order). Every thread works out the weights itself, so no thread waits for
// another. The 64 fp16 results go to the head's 32 words of `out`: lanes d and d ^ 1 of one wave
// share a word.
template <typename Get>
__device__ __forceinline__ void combine_store(int ns, int d, uint64_t* out, unsigned tag, Get get) {
  constexpr int S = kMaxCombineSplits;
  // every split's values first (get may read LDS: one batch of reads, not one round trip per split)
  float pm[S], pl[S], pa[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    get(s, pm[s], pl[s], pa[s]);
    if (s >= ns) {
      pm[s] = -INFINITY;
      pl[s] = pa[s] = 0.f;
    }
  }
  float m = -INFINITY;
#pragma unroll
  for (int s = 0; s < S; ++s) m = fmaxf(m, pm[s]);
  float den = 0.f, num = 0.f;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const float w = pl[s] > 0.f ? __expf(pm[s] - m) : 0.f;
    den = fmaf(pl[s], w, den);
    num = w != 0.f ? fmaf(pa[s], w, num) : num;
  }
  const unsigned lo = half_bits(f2h(num / den));
  const unsigned hi = static_cast<unsigned>(__builtin_amdgcn_ds_swizzle(static_cast<int>(lo), 0x041F));  // lane ^ 1
  if ((d & 1) == 0) ll_store(out + d / 2, tag, lo | (hi << 16));
}

// One head's attention output from its split partials in LDS (part[s * kPartWords + d], d < 64 the value
// sums, then m and l), by threads d < 64 (combine_store). All threads of the block call it: its
// barrier frees part for the caller.
__device__ __forceinline__ void head_combine(const float* part, int ns, int head, uint64_t* out, unsigned tag) {
  const int tid = threadIdx.x;
  if (tid < kHeadDim)
    combine_store(ns, tid, out + head * 32, tag, [&](int s, float& m, float& l, float& a) {
      m = part[s * kPartWords + kHeadDim];
      l = part[s * kPartWords + kHeadDim + 1];
      a = part[s * kPartWords + tid];
    });
  __syncthreads();  // part is free again
}

// head_combine for NV vectors at once (the prompt pass): vector v's partials at part[v S kPartWords ..],
// S = kMaxCombineSplits; 128 threads per vector run head_combine's arithmetic for it, so each vector's
// output is what head_combine gives.
template <int NV>
__device__ __forceinline__ void head_combine_nv(const float* part, int ns, int head, float* wgt, float* den_lds,
                                                uint64_t* out, unsigned tag) {
  constexpr int S = kMaxCombineSplits;
  static_assert(NV * 128 <= kStepThreads && NV <= kMaxCombineHeads, "one 128-thread group per vector");
  const int tid = threadIdx.x, v = tid >> 7, t = tid & 127;
  const float* vp = part + v * S * kPartWords;
  if (v < NV && t == 0) {
    float pm[S], pl[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      pm[s] = s < ns ? vp[s * kPartWords + kHeadDim] : -INFINITY;
      pl[s] = s < ns ? vp[s * kPartWords + kHeadDim + 1] : 0.f;
    }
    float m = -INFINITY;
#pragma unroll
    for (int s = 0; s < S; ++s) m = fmaxf(m, pm[s]);
    float den = 0.f;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const float w = pl[s] > 0.f ? __expf(pm[s] - m) : 0.f;
      wgt[v * S + s] = w;
      den = fmaf(pl[s], w, den);
    }
    den_lds[v] = den;
  }
  __syncthreads();
  if (v < NV && t < kHeadDim) {  // one whole wave per vector: the lane ^ 1 swizzle pairs stay inside it
    float num = 0.f;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const float pa = s < ns ? vp[s * kPartWords + t] : 0.f;
      if (wgt[v * S + s] != 0.f) num = fmaf(pa, wgt[v * S + s], num);
    }
    const unsigned lo = half_bits(f2h(num / den_lds[v]));
    const unsigned hi = static_cast<unsigned>(__builtin_amdgcn_ds_swizzle(static_cast<int>(lo), 0x041F));  // lane ^ 1
    if ((t & 1) == 0) ll_store(out + v * kVecWords + head * 32 + t / 2, tag, lo | (hi << 16));
  }
  __syncthreads();  // part, wgt and den are free again
}

// The q (and fresh k, v) words of one head: threads t < 96 fetch word t % 32 of part t / 32 (q, k, v;
// parts with want[p] false are skipped) into q_lds[p][...].
__device__ __forceinline__ void fetch_head_vectors(const uint64_t* qsrc, int head, bool want_kv, uint4 (*q_lds)[8],
                                                   const Ll& c) {
  const int tid = threadIdx.x, part_sel = tid >> 5, word = tid & 31;
  int idx[1] = {-1};
  if (part_sel == 0 || (want_kv && part_sel < 3)) idx[0] = part_sel * kVecWords + head * 32 + word;
  unsigned v[1];
  ll_wait<1>(qsrc, idx, v, c);
  if (idx[0] >= 0) reinterpret_cast<unsigned*>(&q_lds[part_sel][0])[word] = v[0];
}

// Self attention of one head in one block, every split of 64 keys (reference split kernel arithmetic,
// attn_split_kernel<2, false>: waves 0-3 take splits 0, 2, 4, 6, waves 4-7 splits 1, 3, 5, 7), the
// split partials kept in LDS and combined in the block: no partial leaves the CU. The head's K/V rows
// are requested before its query is awaited; the fresh K/V row (position pos) is written to the cache
// and used in place of the cached one. With NV vectors per phase (the prompt pass, positions pos0 ..
// pos0 + NV - 1) the block runs query z at position pos0 + z: the fresh rows of vectors 0 .. z stand in
// for cache rows pos0 .. pos0 + z (the cache rows of the other vectors are written by other blocks of
// the same phase), as the batched split kernel does.
template <int NV = 1>
__device__ __forceinline__ void self_attn_head(const Ll& c, int head, int z, int ns, _Float16* kc, _Float16* vc,
                                               int max_len, int pos0, const uint64_t* qkv, uint64_t* out, float scale,
                                               AttnLds& s, float* part, float* wave_slots, uint4 (*kvf)[2][8],
                                               const Tl& tl, int tl_slot) {
  constexpr int MAXP = 2, kRounds = kMaxCombineSplits / 2;
  const int pos = NV == 1 ? pos0 : min(pos0 + z, max_len - 1);  // as the batched split kernel clamps it
  // an opaque copy of the thread index: the addresses derived from it are computed here, not hoisted
  // to the kernel's start and kept (spilled) across the layers
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63, wave = tid >> 6, half = wave >> 2, hw = wave & 3;
  const int t4 = tid & 255, ks = lane >> 3, cc = lane & 7;
  const size_t hoff = static_cast<size_t>(head) * max_len * kHeadDim;
  uint4 kr[kRounds][MAXP], vr[kRounds][MAXP];
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int split = half + 2 * r, begin = split * kSelfSplitKeys;
    const int w0 = begin + hw * MAXP * 8;
    const int wend = min(min(w0 + MAXP * 8, begin + kSelfSplitKeys), max_len);
#pragma unroll
    for (int p = 0; p < MAXP; ++p) {
      // Rows past the position are never read: a later step of the same launch writes them, and an
      // earlier read could leave a stale copy in this CU's caches. A key that is not the split's (past
      // the position or wend, or in a split past ns) loads row min(j, wend - 1, pos) instead and is
      // masked in split_wave_partial: no load sits under a lane mask (the join after one waits for
      // every earlier load).
      const int j = max(0, min(min(w0 + p * 8 + ks, wend - 1), pos));
      kr[r][p] = reinterpret_cast<const uint4*>(kc + hoff + static_cast<size_t>(j) * kHeadDim)[cc];
      vr[r][p] = reinterpret_cast<const uint4*>(vc + hoff + static_cast<size_t>(j) * kHeadDim)[cc];
    }
  }
  if constexpr (NV == 1) {
    fetch_head_vectors(qkv, head, true, s.q[0], c);
  } else {  // query z, then the fresh k and v rows of vectors 0 .. z (the q/k/v words of vector v at v * 1920)
    int idx[1] = {-1};
    unsigned* dst = nullptr;
    if (tid < 32) {
      idx[0] = z * kQkvWords + head * 32 + tid;
      dst = reinterpret_cast<unsigned*>(&s.q[0][0][0]) + tid;
    } else if (tid < 32 + 64 * (z + 1)) {
      const int t = tid - 32, vv = t >> 6, kv = (t >> 5) & 1, word = t & 31;
      idx[0] = vv * kQkvWords + (1 + kv) * kVecWords + head * 32 + word;
      dst = reinterpret_cast<unsigned*>(&kvf[vv][kv][0]) + word;
    }
    unsigned v[1];
    ll_wait<1>(qkv, idx, v, c);
    if (idx[0] >= 0) *dst = v[0];
  }
  __syncthreads();
  tl.mark(tl_slot + 1);
  if (tid < 16) {  // the fresh row into the cache, for the steps that follow
    if constexpr (NV == 1) {
      if (tid < 8)
        reinterpret_cast<uint4*>(kc + hoff + static_cast<size_t>(pos) * kHeadDim)[tid] = s.q[0][1][tid];
      else
        reinterpret_cast<uint4*>(vc + hoff + static_cast<size_t>(pos) * kHeadDim)[tid - 8] = s.q[0][2][tid - 8];
    } else {
      if (tid < 8)
        reinterpret_cast<uint4*>(kc + hoff + static_cast<size_t>(pos) * kHeadDim)[tid] = kvf[z][0][tid];
      else
        reinterpret_cast<uint4*>(vc + hoff + static_cast<size_t>(pos) * kHeadDim)[tid - 8] = kvf[z][1][tid - 8];
    }
  }
  const uint4 qc = s.q[0][0][cc];
  const bool tl0 = tl_slot == tl_phase(0, 2);
  if (tl0) tl.mark(kTlSa + kTlSaRow);
  if constexpr (NV == 1) {
    // Every round's wave partials into slots of their own (split s, wave hw), so the rounds run back to
    // back without a barrier; then one merge step. Each split's (m, l, acc) is split_merge<4> of its four
    // wave partials and the head's output combine_store over the splits, as in the rounds below.
    float* wm = wave_slots;                                 // [kMaxCombineSplits][4]
    float* wl = wave_slots + kMaxCombineSplits * 4;         // [kMaxCombineSplits][4]
    float* wacc = wave_slots + 2 * kMaxCombineSplits * 4;   // [kMaxCombineSplits][4][64]
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      if (2 * r >= ns) break;  // block-uniform
      const int split = half + 2 * r, begin = split * kSelfSplitKeys;
      const int w0 = begin + hw * MAXP * 8;
      const int wend = min(min(w0 + MAXP * 8, begin + kSelfSplitKeys), max_len);
      const int n = min(kSelfSplitKeys, pos + 1 - begin);
      if (split < ns) {
#pragma unroll
        for (int p = 0; p < MAXP; ++p)
          if (w0 + p * 8 + ks == pos) {  // the new row replaces the (stale) cached one
            kr[r][p] = s.q[0][1][cc];
            vr[r][p] = s.q[0][2][cc];
          }
        split_wave_partial<MAXP>(kr[r], vr[r], qc, w0, min(wend, begin + n), scale, &wm[split * 4 + hw],
                                 &wl[split * 4 + hw], wacc + (split * 4 + hw) * kHeadDim);
      }
    }
    if (tl0) tl.mark_wave(kTlWave);
    if (tl0) tl.mark(kTlSa + kTlSaPartial);
    __syncthreads();
    if (tl0) tl.mark(kTlSa + kTlSaBarrier);
    using WaccRow = const float (*)[kHeadDim];
    if (ns <= 2) {  // block-uniform: thread d merges both splits itself and combines them, no second barrier
      if (tid < kHeadDim) {
        float m0, l0, o0, m1 = -INFINITY, l1 = 0.f, o1 = 0.f;
        split_merge<4>(wm, wl, reinterpret_cast<WaccRow>(wacc), tid, m0, l0, o0);
        if (ns > 1) split_merge<4>(wm + 4, wl + 4, reinterpret_cast<WaccRow>(wacc + 4 * kHeadDim), tid, m1, l1, o1);
        if (tl0) tl.mark(kTlSa + kTlSaMerged);
        combine_store(ns, tid, out + head * 32, c.tag, [&](int sp, float& m, float& l, float& a) {
          m = sp == 0 ? m0 : m1;
          l = sp == 0 ? l0 : l1;
          a = sp == 0 ? o0 : o1;
        });
      }
      tl.mark(tl_slot + 3);
      __syncthreads();  // the slots and part are free again
    } else {  // thread (split, d) merges, then the combine
      const int sp = tid >> 6, d = tid & 63;
      if (sp < ns) {
        float m, l, o;
        split_merge<4>(wm + sp * 4, wl + sp * 4, reinterpret_cast<WaccRow>(wacc + sp * 4 * kHeadDim), d, m, l, o);
        part[sp * kPartWords + d] = o;
        if (d == 0) {
          part[sp * kPartWords + kHeadDim] = m;
          part[sp * kPartWords + kHeadDim + 1] = l;
        }
      }
      __syncthreads();
      if (tl0) tl.mark(kTlSa + kTlSaMerged);
      tl.mark(tl_slot + 3);
      head_combine(part, ns, head, out, c.tag);
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    if (2 * r >= ns) break;  // block-uniform
    const int split = half + 2 * r, begin = split * kSelfSplitKeys;
    const bool act = split < ns;
    const int w0 = begin + hw * MAXP * 8;
    const int wend = min(min(w0 + MAXP * 8, begin + kSelfSplitKeys), max_len);
    const int n = min(kSelfSplitKeys, pos + 1 - begin);
    if (act) {
#pragma unroll
      for (int p = 0; p < MAXP; ++p) {
        const int j = w0 + p * 8 + ks;
        if constexpr (NV == 1) {
          if (w0 + p * 8 + ks == pos) {  // the new row replaces the (stale) cached one
            kr[r][p] = s.q[0][1][cc];
            vr[r][p] = s.q[0][2][cc];
          }
        } else if (j == pos) {  // this vector's fresh row
          kr[r][p] = kvf[z][0][cc];
          vr[r][p] = kvf[z][1][cc];
        } else if (j >= pos0 && j < pos) {  // an earlier vector's fresh row
          kr[r][p] = kvf[j - pos0][0][cc];
          vr[r][p] = kvf[j - pos0][1][cc];
        }
      }
      split_wave_partial<MAXP>(kr[r], vr[r], qc, w0, min(wend, begin + n), scale, &s.wm[half][hw], &s.wl[half][hw],
                               s.wacc[half][hw]);
    }
    if (tl0 && r == 0) tl.mark(kTlSa + kTlSaPartial);
    __syncthreads();
    if (act && t4 < kHeadDim) {
      float m, l, o;
      split_merge<4>(s.wm[half], s.wl[half], s.wacc[half], t4, m, l, o);
      part[split * kPartWords + t4] = o;
      if (t4 == 0) {
        part[split * kPartWords + kHeadDim] = m;
        part[split * kPartWords + kHeadDim + 1] = l;
      }
    }
    __syncthreads();
    if (tl0 && r == 0) tl.mark(kTlSa + kTlSaMerged);
  }
  tl.mark(tl_slot + 3);
  head_combine(part, ns, head, NV == 1 ? out : out + z * kVecWords, c.tag);
}

// Cross-attention split items for one query, one item per block at a time: waves 0-3 run it exactly as
// attn_split_kernel<8, false, 4> runs one block (one wave per SIMD; waves 4-7 only keep the barriers) and
// store its partial (66 words, one coalesced store). Item k of the phase is split k % (nsplit - 1) of head
// k / (nsplit - 1) for k < 20 (nsplit - 1), then the last split of head k - 20 (nsplit - 1); a block takes
// items rank, rank + workers, ... The block that ran a head's last split then collects the head's
// partials and combines them, so the combining blocks end the run and the phase after the cross-out can
// reuse the run's first blocks. A block reaches its last-split items only after its other items, so no
// wait depends on a block that is itself waiting.
__device__ __forceinline__ void cross_attn_items(const Ll& c, int rank, int workers, int nsplit, const _Float16* kc,
                                                 const _Float16* vc, int max_len, const uint64_t* qsrc,
                                                 uint64_t* part_g, uint64_t* out, float scale, AttnLds& s, float* part,
                                                 const Tl& tl, int tl_slot) {
  constexpr int MAXP = FW_ATTN256_P, kNW = kCrossSplitKeys / (8 * MAXP), kKeys = kCrossSplitKeys;
  static_assert(kNW <= kStepWaves && kNW <= 8, "one item's waves in a block");
  const int tid = threadIdx.x, lane = tid & 63, ks = lane >> 3, cc = lane & 7;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar branches, no lane masks
  float* wm = &s.wm[0][0];            // [8] (the two halves' slots, contiguous)
  float* wl = &s.wl[0][0];
  float* wacc = &s.wacc[0][0][0];     // [8][64]
  const int nitems = kStepHeads * nsplit, n_first = kStepHeads * (nsplit - 1);
  for (int k = rank; k < nitems; k += workers) {  // block-uniform
    const bool last = k >= n_first;
    const int head = last ? k - n_first : k / (nsplit - 1), split = last ? nsplit - 1 : k % (nsplit - 1);
    const size_t hoff = static_cast<size_t>(head) * max_len * kHeadDim;
    const int begin = split * kKeys;
    const int n = min(kKeys, max_len - begin);
    const int w0 = begin + (wave % kNW) * MAXP * 8;
    const int wend = min(min(w0 + MAXP * 8, begin + kKeys), max_len);
    uint4 kr[MAXP], vr[MAXP];
    if (wave < kNW) {
#pragma unroll
      for (int p = 0; p < MAXP; ++p) {
        // keys past wend load row wend - 1 and are masked: no load under a lane mask
        const int j = max(0, min(w0 + p * 8 + ks, wend - 1));
        kr[p] = reinterpret_cast<const uint4*>(kc + hoff + static_cast<size_t>(j) * kHeadDim)[cc];
        vr[p] = reinterpret_cast<const uint4*>(vc + hoff + static_cast<size_t>(j) * kHeadDim)[cc];
      }
    }
    {  // the head's query: 32 words
      int idx[1] = {tid < 32 ? head * 32 + tid : -1};
      unsigned v[1];
      ll_wait<1>(qsrc, idx, v, c);
      if (idx[0] >= 0) reinterpret_cast<unsigned*>(&s.q[0][0][0])[tid] = v[0];
    }
    __syncthreads();
    if (k == rank) tl.mark(tl_slot + 1);
    if (wave < kNW && n > 0)
      split_wave_partial<MAXP>(kr, vr, s.q[0][0][cc], w0, min(wend, begin + n), scale, wm + wave, wl + wave,
                               wacc + wave * kHeadDim);
    __syncthreads();
    if (tid < kPartWords) {
      float m = -INFINITY, l = 0.f, o = 0.f;
      if (n > 0)
        split_merge<kNW>(wm, wl, reinterpret_cast<const float(*)[kHeadDim]>(wacc), tid < kHeadDim ? tid : 0, m, l, o);
      const float val = tid < kHeadDim ? o : (tid == kHeadDim ? m : l);
      ll_store(part_g + static_cast<size_t>(split * kStepHeads + head) * kPartWords + tid, c.tag, __float_as_uint(val));
    }
    __syncthreads();  // s is reused below
    tl.mark(tl_slot + 2);
    if (last) {  // block-uniform: collect the head's partials and combine
      int idx[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int t = tid + q * kStepThreads;
        idx[q] = t < nsplit * kPartWords ? ((t / kPartWords) * kStepHeads + head) * kPartWords + t % kPartWords : -1;
      }
      unsigned v[2];
      ll_wait<2>(part_g, idx, v, c);
#pragma unroll
      for (int q = 0; q < 2; ++q)
        if (idx[q] >= 0) part[tid + q * kStepThreads] = __uint_as_float(v[q]);
      __syncthreads();
      head_combine(part, nsplit, head, out, c.tag);
      tl.mark(tl_slot + 3);
    }
  }
}

// split_wave_partial for NV queries on the same K/V registers, their steps interleaved so the
// cross-lane reductions of the NV queries overlap. Each query's arithmetic is split_wave_partial's:
// a query whose keys are all masked gets p = 0 for every key (split_wave_partial skips them), so its
// sums are the same zeros.
template <int MAXP, int NV>
__device__ __forceinline__ void split_wave_partial_nv(const uint4 (&kr)[MAXP], const uint4 (&vr)[MAXP],
                                                      const uint4* const (&q)[NV], int w0, int w1, float scale,
                                                      float* const (&wm)[NV], float* const (&wl)[NV],
                                                      float* const (&wacc_row)[NV]) {
  const int lane = threadIdx.x & 63, ks = lane >> 3, c = lane & 7;
  float sc[NV][MAXP], mx[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const uint4 qc = *q[v];
    mx[v] = -INFINITY;
#pragma unroll
    for (int p = 0; p < MAXP; ++p) {
      sc[v][p] = group_sum<8>(dot8(kr[p], qc, 0.f)) * scale;
      if (w0 + p * 8 + ks >= w1) sc[v][p] = -INFINITY;
      mx[v] = fmaxf(mx[v], sc[v][p]);
    }
  }
#pragma unroll
  for (int v = 0; v < NV; ++v) mx[v] = group_max<64>(mx[v]);
  float acc[NV][8], psum[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    psum[v] = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[v][t] = 0.f;
  }
#pragma unroll
  for (int p = 0; p < MAXP; ++p) {
    const h2v* v2 = reinterpret_cast<const h2v*>(&vr[p]);
    const bool live = w0 + p * 8 + ks < w1;  // a masked key's V counts as zero, as in split_wave_partial
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const float pj = mx[v] != -INFINITY ? __expf(sc[v][p] - mx[v]) : 0.f;
      psum[v] += pj;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        acc[v][2 * t] = fmaf(pj, live ? h2f(v2[t].x) : 0.f, acc[v][2 * t]);
        acc[v][2 * t + 1] = fmaf(pj, live ? h2f(v2[t].y) : 0.f, acc[v][2 * t + 1]);
      }
    }
  }
  float o[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    psum[v] = xor_add<32>(xor_add<16>(xor_add<8>(psum[v])));
    o[v] = sum8_transposed(acc[v]);
  }
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    if (lane == 0) {
      *wm[v] = mx[v];
      *wl[v] = psum[v];
    }
    wacc_row[v][c * 8 + sum8_index(lane)] = o[v];
  }
}

// Cross attention for NV query vectors (the prompt pass): item i is (head i / nsplit, split i % nsplit)
// as for one vector; its K/V rows are loaded once and every vector's query runs on them, each with
// attn_split_kernel's arithmetic. Vector v's partials and output lie in regions of their own.
template <int NV>
struct AttnNvLds {
  float wm[NV][2][4], wl[NV][2][4];
  float wacc[NV][2][4][kHeadDim];
  uint4 q[2][NV][8];
};

template <int NV>
__device__ __forceinline__ void cross_attn_items_nv(const Ll& c, int rank, int workers, int nitems, int nsplit,
                                                    const _Float16* kc, const _Float16* vc, int max_len,
                                                    const uint64_t* qsrc, uint64_t* part_g, uint64_t* out,
                                                    float scale, AttnNvLds<NV>& s, float* part, float* wgt,
                                                    float* den) {
  constexpr int MAXP = 8, kKeys = kCrossSplitKeys;
  static_assert(sizeof(AttnNvLds<NV>) >= NV * kMaxCombineSplits * kPartWords * sizeof(float),
                "the combine's partials fit the operand space");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = wave >> 2, hw = wave & 3;
  const int t4 = tid & 255, ks = lane >> 3, cc = lane & 7;
  for (int base = 2 * rank; base < nitems; base += 2 * workers) {  // block-uniform
    const int item = base + half;
    const bool act = item < nitems;
    const int head = act ? item / nsplit : 0, split = act ? item % nsplit : 0;
    const size_t hoff = static_cast<size_t>(head) * max_len * kHeadDim;
    const int begin = split * kKeys;
    const int w0 = begin + hw * MAXP * 8;
    const int wend = min(min(w0 + MAXP * 8, begin + kKeys), max_len);
    const int n = min(kKeys, max_len - begin);
    uint4 kr[MAXP], vr[MAXP];
#pragma unroll
    for (int p = 0; p < MAXP; ++p) {
      // keys past wend (and an idle half's) load row wend - 1 and are masked: no load under a lane mask
      const int j = max(0, min(w0 + p * 8 + ks, wend - 1));
      kr[p] = reinterpret_cast<const uint4*>(kc + hoff + static_cast<size_t>(j) * kHeadDim)[cc];
      vr[p] = reinterpret_cast<const uint4*>(vc + hoff + static_cast<size_t>(j) * kHeadDim)[cc];
    }
    {  // the head's queries: 32 words per vector and half
      int idx[1] = {act && t4 < 32 * NV ? (t4 >> 5) * kVecWords + head * 32 + (t4 & 31) : -1};
      unsigned v[1];
      ll_wait<1>(qsrc, idx, v, c);
      if (idx[0] >= 0) reinterpret_cast<unsigned*>(&s.q[half][t4 >> 5][0])[t4 & 31] = v[0];
    }
    __syncthreads();
    if (act && n > 0) {
      const uint4* q[NV];
      float* wm[NV];
      float* wl[NV];
      float* wa[NV];
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        q[v] = &s.q[half][v][cc];
        wm[v] = &s.wm[v][half][hw];
        wl[v] = &s.wl[v][half][hw];
        wa[v] = s.wacc[v][half][hw];
      }
      split_wave_partial_nv<MAXP, NV>(kr, vr, q, w0, min(wend, begin + n), scale, wm, wl, wa);
    }
    __syncthreads();
    if (act) {
      for (int w = t4; w < NV * kPartWords; w += 256) {
        const int v = w / kPartWords, e = w % kPartWords;
        float m = -INFINITY, l = 0.f, o = 0.f;
        if (n > 0) split_merge<4>(s.wm[v][half], s.wl[v][half], s.wacc[v][half], e < kHeadDim ? e : 0, m, l, o);
        const float val = e < kHeadDim ? o : (e == kHeadDim ? m : l);
        ll_store(part_g + static_cast<size_t>(v) * kPartRegion + static_cast<size_t>(split * kStepHeads + head) * kPartWords +
                     e,
                 c.tag, __float_as_uint(val));
      }
    }
    __syncthreads();  // s is reused below
    // heads whose last split this block ran: collect each vector's partials and combine
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int it = base + hf;
      if (it >= nitems || it % nsplit != nsplit - 1) continue;  // block-uniform
      const int h = it / nsplit;
      // every vector's partials of the head in one wait, into the operand space of s (free here)
      constexpr int kPer = (NV * kMaxCombineSplits * kPartWords + kStepThreads - 1) / kStepThreads;
      float* pall = reinterpret_cast<float*>(&s);
      const int per_v = nsplit * kPartWords;
      int idx[kPer], dst[kPer];
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        const int t = tid + k * kStepThreads, v = t / per_v, r = t - v * per_v;
        const bool ok = v < NV;
        idx[k] = ok ? v * kPartRegion + ((r / kPartWords) * kStepHeads + h) * kPartWords + r % kPartWords : -1;
        dst[k] = ok ? v * kMaxCombineSplits * kPartWords + r : -1;
      }
      unsigned pv[kPer];
      ll_wait<kPer>(part_g, idx, pv, c);
#pragma unroll
      for (int k = 0; k < kPer; ++k)
        if (dst[k] >= 0) pall[dst[k]] = __uint_as_float(pv[k]);
      __syncthreads();
      head_combine_nv<NV>(pall, nsplit, h, wgt, den, out, c.tag);
    }
  }
}

// An attention output vector (640 words: 20 heads of 32, each head written by one store) into x_lds:
// one sentinel per head, then every word.
__device__ __forceinline__ void fetch_attn_vector(const uint64_t* src, _Float16* x_lds, const Ll& c) {
  const int tid = threadIdx.x;
  const int idx[2] = {tid < kVecWords ? tid : -1, tid + kStepThreads < kVecWords ? tid + kStepThreads : -1};
  unsigned v[2];
  ll_wait<2>(src, idx, v, c);
#pragma unroll
  for (int k = 0; k < 2; ++k)
    if (idx[k] >= 0) reinterpret_cast<unsigned*>(x_lds)[idx[k]] = v[k];
}

// NV attention output vectors (640 words apart) into x_lds (1280 halves apart).
template <int NV>
__device__ __forceinline__ void fetch_attn_vectors(const uint64_t* src, _Float16* x_lds, const Ll& c) {
  if constexpr (NV == 1) {
    fetch_attn_vector(src, x_lds, c);
  } else {
    constexpr int kWords = NV * kVecWords, kPer = (kWords + kStepThreads - 1) / kStepThreads;
    const int tid = threadIdx.x;
    int idx[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) idx[k] = tid + k * kStepThreads < kWords ? tid + k * kStepThreads : -1;
    unsigned v[kPer];
    ll_wait<kPer>(src, idx, v, c);
#pragma unroll
    for (int k = 0; k < kPer; ++k)
      if (idx[k] >= 0) reinterpret_cast<unsigned*>(x_lds)[idx[k]] = v[k];
  }
}

// ---------------------------------------------------------------------------------------------
// Final LayerNorm + LM head with the int8 pre-pass + argmax + finalize (the arithmetic of
// lm_head_q8_kernel<true> and argmax_finalize_kernel in decode.hip). Every block scores a contiguous
// share of the int8 table (the candidate rule holds for any partition of the rows into blocks), part of
// it held in LDS, rescores its candidates on the fp16 table with lm_head_kernel's lane split and order,
// and hands its packed maximum to the last block as two tagged words; that block takes the maximum,
// finalizes and broadcasts the token, position and count to every block for the next step. (Every
// block gathering the maxima itself, with no broadcast, measured 2.6 us slower a step: 256 blocks
// polling 512 words each load the memory system while the last blocks still score.)
// ---------------------------------------------------------------------------------------------
constexpr int kLmRowWaves = kStepWaves - 1;                    // waves 0-6 score rows, wave 7 awaits the
constexpr int kLmBatchRows = kLmRowWaves * (kWave / kQ8Lpr);  // last fc2 output; 28 rows a batch, 4 a wave
constexpr int kLmMaxBatches = 8;                              // per block: ceil(vocab / G) <= 8 * 28
// Batches in flight per wave, requested when the block arrives and refilled as they are scored. Two
// measured best: requested deeper (4, 6) or earlier than the block's arrival here, the table loads slow
// the last fc2 and the stream itself down (4 with the resident rows too: 105.0 against 103.1 us a step).
#ifndef FW_LM_BUFS
#define FW_LM_BUFS 2
#endif
#ifndef FW_EMBED_WARM
#define FW_EMBED_WARM 1
#endif
#ifndef FW_LM_CATCH_FIRST
#define FW_LM_CATCH_FIRST 0  // every block adds the last fc2 output before requesting its table rows
#endif
#ifndef FW_QKV_WARM
#define FW_QKV_WARM 1  // layer 0's q/k/v rows read into L2 while the token is awaited
#endif
constexpr int kLmBufs = FW_LM_BUFS;
static_assert(kLmBufs >= 1 && kLmBufs <= kLmMaxBatches, "FW_LM_BUFS");
constexpr int kMaxGrid = 1024;                                // blocks whose maxima the hand-off region holds
static_assert(kLmMaxBatches * kLmBatchRows <= 256, "candidate list");
// Rows of its share each block keeps in LDS for the whole launch (the last ones of the share): they are
// read from HBM once per launch instead of once per step. The rest of the share streams each step. They
// live in the launch's dynamic LDS, which sits above every static array (a 130 KB static array placed
// first would push the others past the 64 KB reach of the LDS instructions' offset field), laid out as
// n rows of 1280 int8, then n (scale, bound) pairs, then n suppress flags.
#ifndef FW_LM_RES_ROWS
#define FW_LM_RES_ROWS 104
#endif
constexpr int kLmResRows = FW_LM_RES_ROWS;
constexpr int kLmResRowBytes = kHidden + sizeof(float2) + 1;
static_assert(kLmResRows >= 0 && kLmResRows % 4 == 0 && kLmResRows <= kLmMaxBatches * kLmBatchRows,
              "FW_LM_RES_ROWS: whole groups of 4 rows, at most a share");
struct LmResView {
  const uint4* q;
  const float2* meta;
  const uint8_t* sup;
  int rows;  // rows the LDS holds (0: none)
};
__host__ __device__ inline size_t lm_res_bytes(int rows) {
  return (static_cast<size_t>(rows) * kLmResRowBytes + 15) / 16 * 16;
}
extern __shared__ __align__(16) uint4 lm_res_lds[];  // the launch's dynamic LDS
__device__ __forceinline__ LmResView lm_res_view(int rows) {
  const float2* meta = reinterpret_cast<const float2*>(lm_res_lds + rows * kQ8Chunks);
  return {lm_res_lds, meta, reinterpret_cast<const uint8_t*>(meta + rows), rows};
}


struct alignas(16) LmLds {  // yhi / ylo are read as 16-byte chunks
  int8_t yhi[kHidden], ylo[kHidden];
  h2v gamma[kHidden / 2], beta[kHidden / 2];  // the final LayerNorm's, read at the start of the launch
  float ub[kLmMaxBatches * kLmBatchRows];
  int cand[kLmMaxBatches * kLmBatchRows];
  int ncand;
  unsigned long long best[kStepWaves * 2];
  unsigned long long fin[kStepWaves];  // the finalizing block's wave maxima
  int64_t warm[2];                     // the finalizing block's token and next position
};

// y = LN(h_res) with the reduction order of ln_finish<1024, true> (the LM-head kernel's 1024-thread
// block): thread t stands for threads t and t + 512 of that block, whose partial sums go through the
// same wave butterflies and are added over the 16 wave slots in order. h_res is already rounded.
__device__ __forceinline__ void ln_final(const _Float16* h_res, const h2v* g2, const h2v* b2, float eps, _Float16* y,
                                         float* red) {
  constexpr int NT = 1024, kVirt = NT / kStepThreads, kWaves = NT / kWave;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const h2v* h2 = reinterpret_cast<const h2v*>(h_res);
  float2 r[kVirt];
  h2v g[kVirt], be[kVirt];
  float part[kVirt];
#pragma unroll
  for (int k = 0; k < kVirt; ++k) {
    const int vt = tid + k * kStepThreads;
    r[k] = make_float2(0.f, 0.f);
    g[k] = be[k] = {static_cast<_Float16>(0.f), static_cast<_Float16>(0.f)};
    float sum = 0.f;
    if (vt < kHidden / 2) {
      const h2v a = h2[vt];
      const float rx = h2f(a.x), ry = h2f(a.y);
      r[k] = make_float2(rx, ry);
      sum += rx + ry;
      g[k] = g2[vt];
      be[k] = b2[vt];
    }
    part[k] = group_sum<kWave>(sum);
  }
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < kVirt; ++k) red[wave + k * kStepWaves] = part[k];
  }
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) s += red[i];
  const float mean = s * (1.0f / kHidden);
#pragma unroll
  for (int k = 0; k < kVirt; ++k) {
    const int vt = tid + k * kStepThreads;
    float sq = 0.f;
    if (vt < kHidden / 2) {
      const float dx = r[k].x - mean, dy = r[k].y - mean;
      sq += dx * dx + dy * dy;
    }
    part[k] = group_sum<kWave>(sq);
  }
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < kVirt; ++k) red[kWaves + wave + k * kStepWaves] = part[k];
  }
  __syncthreads();
  float s2 = 0.f;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) s2 += red[kWaves + i];
  const float var = s2 * (1.0f / kHidden);
  const float inv = rsqrtf(var + eps);
  h2v* y2 = reinterpret_cast<h2v*>(y);
#pragma unroll
  for (int k = 0; k < kVirt; ++k) {
    const int vt = tid + k * kStepThreads;
    if (vt < kHidden / 2) {
      h2v o;
      o.x = f2h((r[k].x - mean) * inv * h2f(g[k].x) + h2f(be[k].x));
      o.y = f2h((r[k].y - mean) * inv * h2f(g[k].y) + h2f(be[k].y));
      y2[vt] = o;
    }
  }
}

// The block that takes the maximum over the blocks and finalizes: the last one, which the first
// phase of the next step does not use.
__device__ __forceinline__ int fin_block() { return gridDim.x - 1; }

// LM-head rows of blocks 0 .. b - 1: the table split in proportion to block weights, kLmWeight for
// most blocks and kLmLateWeight for the n_late blocks from late0 on (taken round the grid).
#ifndef FW_LM_LATE_WEIGHT
#define FW_LM_LATE_WEIGHT 6  // sevenths of a share for the blocks that ran the last fc2
#endif
constexpr int kLmWeight = 7, kLmLateWeight = FW_LM_LATE_WEIGHT;
static_assert(kLmLateWeight >= 1 && kLmLateWeight <= 14, "FW_LM_LATE_WEIGHT");
__host__ __device__ inline int lm_rows_before(int b, int vocab, int G, int late0, int n_late) {
  const int wrap = late0 + n_late - G;  // late blocks past the end of the grid, counted from block 0
  const int late = (wrap > 0 ? min(b, wrap) : 0) + max(0, min(b, min(G, late0 + n_late)) - late0);
  const int64_t weight = static_cast<int64_t>(kLmWeight) * b - (kLmWeight - kLmLateWeight) * late;
  const int64_t total = static_cast<int64_t>(kLmWeight) * G - (kLmWeight - kLmLateWeight) * n_late;
  return static_cast<int>(static_cast<int64_t>(vocab) * weight / total);
}

// Blocks per phase run: the phases with many rows use every block the previous phase did not, except
// LN3+fc1, which also takes the first half of the cross-attention run (those blocks end their items
// early; the combining blocks are the run's last). At 256 CUs: LN1+q/k/v 176 blocks, self attention 20
// (of a run of 176), out 80, LN2+cross-q 80, cross attention 120, cross-out 80, LN3+fc1 116, fc2 80.
struct StepWorkers {
  int qkv, vec, cross, fc1;
};
__device__ __forceinline__ StepWorkers step_workers(int G) {
  const int vec = min(kVecWorkers, max(1, G * 5 / 16));
  const int cross = min(kCrossWorkers, max(1, G * 15 / 32));
  return {max(1, G - vec), vec, cross, max(1, G - vec - cross / 2)};
}

// The block's share [r0, r1) of the LM-head table: the blocks that ran the last fc2 start last and take
// kLmLateWeight / kLmWeight of the others' share. The schedule's runs start at block 0 each step and
// advance by the same worker counts in every layer, so the share is the same in every step of a launch.
struct LmShare {
  int r0, r1;
  bool late;  // the block ran the last fc2
};
__device__ __forceinline__ LmShare lm_share(int vocab, int n_layers) {
  const int G = gridDim.x;
  const StepWorkers w = step_workers(G);
  const int adv = (2 * w.qkv + 4 * w.vec + w.cross + w.fc1) % G;  // a layer's eight runs
  const int late0 = ((n_layers * adv) % G - w.vec + G) % G;       // the last fc2's run
  const int b = blockIdx.x;
  return {lm_rows_before(b, vocab, G, late0, w.vec), lm_rows_before(b + 1, vocab, G, late0, w.vec),
          (b - late0 + G) % G < w.vec};
}

// With NV vectors (the prompt pass) the LM head scores the last one, at position pos_raw + NV - 1. The
// last rows of the share are read from LDS, loaded there at the start of the launch.
template <int NV = 1>
__device__ __forceinline__ void lm_head_phase(const StepArgs& a, const StepHead& H, const Ll& c, _Float16* h_res,
                                              int& applied, uint64_t* regions, uint64_t* maxima, uint64_t* bcast,
                                              _Float16* y_lds, float* red, LmLds& s, const StepPos& sp,
                                              int64_t n_tok, const Tl& tl) {
  constexpr int NT = 1024, kWaves = NT / kWave;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = gridDim.x, b = blockIdx.x;
  const int sub = lane & (kQ8Lpr - 1), rsel = lane / kQ8Lpr;
  const int wv = __builtin_amdgcn_readfirstlane(wave);  // branches on it are wave-uniform
  // the block's rows: a contiguous share [r0, r1) of the table; rows [r0, rb) stream from HBM in batches
  // of kLmBatchRows, rows [rb, r1) are resident in LDS
  const LmShare share = lm_share(a.vocab, a.n_layers);  // recomputed: nothing stays live across the layers
  const LmResView res = lm_res_view(NV == 1 ? a.lm_res_rows : 0);
  const int r0 = share.r0, r1 = share.r1;
  const int n_res = min(res.rows, r1 - r0);
  const int rb = r1 - n_res;
  const int nb = (rb - r0 + kLmBatchRows - 1) / kLmBatchRows;  // <= kLmMaxBatches
  auto base_of = [&](int k) { return r0 + k * kLmBatchRows; };
  const uint4* wq4 = reinterpret_cast<const uint4*>(H.wq);
  struct Batch {
    uint4 w[kQ8C];
    float2 m;
    uint32_t sp;
  };
  auto load = [&](int k, Batch& bt) {  // rows past rb load row rb - 1 and are dropped when scored
    const size_t row = min(base_of(k) + wave * 4 + rsel, rb - 1);
#pragma unroll
    for (int cc = 0; cc < kQ8C; ++cc) bt.w[cc] = ld_lm_head(wq4 + row * kQ8Chunks + sub + kQ8Lpr * cc);
    bt.m = H.meta[row];
    bt.sp = H.suppress[row];
  };
  if (tid == 0) s.ncand = 0;
  // Waves 0-6 request their first batches as soon as the block gets here (its layer work is done, the
  // last fc2 output may be microseconds away); wave 7 alone awaits the missing residual contributions,
  // so its polls do not queue behind the table loads (a wave's loads return in order).
  constexpr int kBufs = kLmBufs;
  Batch bt[kBufs];
  tl.mark(kTlLm + kTlArrive);
  if (FW_LM_CATCH_FIRST || share.late) {  // block-uniform
    // The blocks that ran the last fc2 arrive last, when its output is already stored: every thread adds
    // it first (one poll round, not queued behind this block's table loads), then the table is requested.
    resid_catch_up<kStepThreads, NV, NV - 1>(h_res, applied, 3 * a.n_layers + 1, regions, a, c, sp);
    if (wv < kLmRowWaves) {
#pragma unroll
      for (int k = 0; k < kBufs; ++k)
        if (k < nb) load(k, bt[k]);
    }
  } else if (wv < kLmRowWaves) {
#pragma unroll
    for (int k = 0; k < kBufs; ++k)
      if (k < nb) load(k, bt[k]);
  } else {
    resid_catch_up<kWave, NV, NV - 1>(h_res, applied, 3 * a.n_layers + 1, regions, a, c, sp, lane);
  }
  applied = 3 * a.n_layers + 1;
  tl.mark(kTlLm + kTlCaught);  // thread 0: wave 0's part (every contribution added in its waves)
  __syncthreads();
  ln_final(h_res + (NV - 1) * kHidden, s.gamma, s.beta, H.eps, y_lds, red);
  __syncthreads();
  tl.mark(kTlLm + kTlY);
  if (H.y_out && b == 0)
    for (int i = tid; i < kHidden / 2; i += kStepThreads)
      reinterpret_cast<unsigned*>(H.y_out)[i] = reinterpret_cast<const unsigned*>(y_lds)[i];
  // y statistics (max |y| and |y|^2, each thread standing for threads t and t + 512 of the 1024-thread
  // block), then y_int = rint(y / t) in two int8 digits
  float wmax[2], wsq[2];
  h2v yp[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int vt = tid + k * kStepThreads;
    yp[k] = {static_cast<_Float16>(0.f), static_cast<_Float16>(0.f)};
    if (vt < kHidden / 2) yp[k] = reinterpret_cast<const h2v*>(y_lds)[vt];
    const float y0 = h2f(yp[k].x), y1 = h2f(yp[k].y);
    wmax[k] = group_max<64>(fmaxf(fabsf(y0), fabsf(y1)));
    wsq[k] = group_sum<64>(y0 * y0 + y1 * y1);
  }
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      red[2 * kWaves + wave + k * kStepWaves] = wmax[k];
      red[3 * kWaves + wave + k * kStepWaves] = wsq[k];
    }
  }
  __syncthreads();
  float amax = 0.f, ysq = 0.f;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    amax = fmaxf(amax, red[2 * kWaves + i]);
    ysq += red[3 * kWaves + i];
  }
  const float tinv = amax > 0.f ? static_cast<float>(kQ8YMax) / amax : 0.f;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int vt = tid + k * kStepThreads;
    if (vt < kHidden / 2) {
      const float y0 = h2f(yp[k].x), y1 = h2f(yp[k].y);
      const int n0 = static_cast<int>(fminf(fmaxf(rintf(y0 * tinv), -kQ8YMax), kQ8YMax));
      const int n1 = static_cast<int>(fminf(fmaxf(rintf(y1 * tinv), -kQ8YMax), kQ8YMax));
      const int h0 = (n0 + 64) >> 7, h1 = (n1 + 64) >> 7;  // floor division; lo digits in [-64, 63]
      s.yhi[2 * vt] = static_cast<int8_t>(h0);
      s.yhi[2 * vt + 1] = static_cast<int8_t>(h1);
      s.ylo[2 * vt] = static_cast<int8_t>(n0 - 128 * h0);
      s.ylo[2 * vt + 1] = static_cast<int8_t>(n1 - 128 * h1);
    }
  }
  __syncthreads();
  tl.mark(kTlLm + kTlDigits);
  const Q8Step q8 = q8_step(amax, ysq);  // the same t as above
  float lb_max = -INFINITY;
  // this lane's chunks of the y digits, read from LDS once for every row it scores (re-reading them per
  // row made the scan bound by LDS bandwidth: 10 of a row's 15 reads)
  uint4 ydh[kQ8C], ydl[kQ8C];
#pragma unroll
  for (int cc = 0; cc < kQ8C; ++cc) {
    ydh[cc] = reinterpret_cast<const uint4*>(s.yhi)[sub + kQ8Lpr * cc];
    ydl[cc] = reinterpret_cast<const uint4*>(s.ylo)[sub + kQ8Lpr * cc];
  }
  // row's bounds into slot row - r0 (rows not in range are scored but neither count nor stored)
  auto score = [&](int row, bool in_range, const Batch& bt) {
    int ah = 0, al = 0;
#pragma unroll
    for (int cc = 0; cc < kQ8C; ++cc) {
      ah = dot16_i8(bt.w[cc], ydh[cc], ah);
      al = dot16_i8(bt.w[cc], ydl[cc], al);
    }
    ah = xor_add_i16(ah);
    al = xor_add_i16(al);
    float ub, lb;
    q8_bounds(ah, al, bt.m, q8, ub, lb);
    const bool live = in_range && !bt.sp;
    ub = live ? ub : -INFINITY;
    lb = live ? lb : -INFINITY;
    lb_max = fmaxf(lb_max, lb);
    if (sub == 0 && in_range) s.ub[row - r0] = ub;
  };
  // HBM batch k (in buffer k % kBufs, refilled once scored)
  auto score_batch = [&](int k, Batch& bt) {
    const int row = base_of(k) + wave * 4 + rsel;
    score(row, row < rb, bt);
    if (k + kBufs < nb) load(k + kBufs, bt);
  };
  if (FW_STEP_TIMELINE && !FW_LM_CATCH_FIRST && wv == 0 && nb > 0) {  // profiling: batch 0 of wave 0 in
    asm volatile("" ::"v"(bt[0].w[kQ8C - 1].x));
    tl.mark(kTlLm + kTlBatch0);
  }
  if (!FW_LM_CATCH_FIRST && wv < kLmRowWaves) {
#pragma unroll
    for (int k = 0; k < kBufs; ++k)
      if (k < nb) score_batch(k, bt[k]);
  }
  tl.mark(kTlLm + kTlRegScored);
  // the resident rows, 4 per wave at a time, by all 8 waves while the next HBM batches are in flight
  // (scoring them first, before batches that arrived at the block long before, measured 1.4 us a step
  // slower; with the batches requested after the catch-up they go first)
  for (int g = wv; 4 * g < n_res; g += kStepWaves) {  // wave-uniform
    const int j = 4 * g + rsel, jc = min(j, n_res - 1);
    Batch rt;
#pragma unroll
    for (int cc = 0; cc < kQ8C; ++cc) rt.w[cc] = res.q[jc * kQ8Chunks + sub + kQ8Lpr * cc];
    rt.m = res.meta[jc];
    rt.sp = res.sup[jc];
    score(rb + j, j < n_res, rt);
  }
  tl.mark(kTlLm + kTlResScored);
  if (wv < kLmRowWaves) {
#pragma unroll
    for (int k = FW_LM_CATCH_FIRST ? 0 : kBufs; k < kLmMaxBatches; ++k)
      if (k < nb) score_batch(k, bt[k % kBufs]);
  }
  tl.mark(kTlLm + kTlScored);
  lb_max = group_max<64>(lb_max);
  if (lane == 0) red[wave] = lb_max;
  __syncthreads();  // also publishes s.ub
  float tb = -INFINITY;
#pragma unroll
  for (int i = 0; i < kStepWaves; ++i) tb = fmaxf(tb, red[i]);
  const float thr = q8_threshold(tb);
  for (int i = tid; i < r1 - r0; i += kStepThreads) {  // every slot of the share was stored above
    const float ub = s.ub[i];
    if (ub != -INFINITY && !(ub < thr)) s.cand[atomicAdd(&s.ncand, 1)] = r0 + i;
  }
  __syncthreads();
  tl.mark(kTlLm + kTlCand);
  // exact logits of the candidates: the lane split and order of lm_head_kernel
  using RS = RowSplit<kHidden>;
  const int sub32 = lane & 31, rsel32 = lane >> 5;
  const uint4* w4 = reinterpret_cast<const uint4*>(H.w);
  uint4 xr[RS::kC];
#pragma unroll
  for (int cc = 0; cc < RS::kC; ++cc) xr[cc] = reinterpret_cast<const uint4*>(y_lds)[sub32 + 32 * cc];
  const int nc = s.ncand;
  unsigned long long mine = 0;
  for (int i0c = wave * 2; i0c < nc; i0c += kStepWaves * 2) {
    const int i = i0c + rsel32;
    const int row = s.cand[i < nc ? i : i0c];
    uint4 wr[RS::kC];
#pragma unroll
    for (int cc = 0; cc < RS::kC; ++cc)
      wr[cc] = ld_lm_head(w4 + static_cast<size_t>(row) * RS::kChunksRow + sub32 + 32 * cc);
    float acc = 0.f;
#pragma unroll
    for (int cc = 0; cc < RS::kC; ++cc) acc = dot8(wr[cc], xr[cc], acc);
    acc = group_sum<32>(acc);
    const unsigned long long sc = pack_score(round_h(acc), row);
    if (i < nc && sc > mine) mine = sc;
  }
  if (sub32 == 0) s.best[wave * 2 + rsel32] = mine;
  __syncthreads();
  if (wv == 0) {  // lanes 0-15 take one slot each, reduced across lanes (no chain of LDS reads)
    unsigned long long m = lane < kStepWaves * 2 ? s.best[lane] : 0ull;
    m = u64_group_max<kStepWaves * 2>(m);
    if (lane == 0) {
      ll_store(maxima + 2 * b, c.tag, static_cast<unsigned>(m));
      ll_store(maxima + 2 * b + 1, c.tag, static_cast<unsigned>(m >> 32));
    }
  }
  tl.mark(kTlLm + kTlMaxStored);
  if (b != fin_block()) return;  // block-uniform
  // the maximum over the blocks (thread i takes block i's two words), then the finalize of
  // argmax_finalize_kernel with the step's state words (only this block writes them), broadcast to
  // every block for the next step as tagged words: token, position, tokens so far, end of the launch
  unsigned long long m = 0;
  for (int i = tid; i < G; i += kStepThreads) {
    const int idx[2] = {2 * i, 2 * i + 1};
    unsigned v[2];
    ll_wait<2>(maxima, idx, v, c);
    const unsigned long long x = (static_cast<unsigned long long>(v[1]) << 32) | v[0];
    m = x > m ? x : m;
  }
  m = u64_group_max<kWave>(m);
  if (lane == 0) s.fin[wave] = m;
  __syncthreads();
  tl.mark(kTlLm + kTlFinGathered);
  if (wv == 0) m = u64_group_max<kStepWaves>(lane < kStepWaves ? s.fin[lane] : 0ull);
  if (tid == 0) {
    const FinArgs fin{H.tokens, a.state, a.cur, a.max_pos};
    const FinOut o = finalize_known(m, n_tok, sp.pos_raw + NV - 1, fin);
    bool stop = false;
    for (int i = 0; i < H.n_eos; ++i) stop = stop || o.tok == H.eos[i];
    ll_store(bcast + 0, c.tag, static_cast<unsigned>(o.tok));
    ll_store(bcast + 1, c.tag, static_cast<unsigned>(o.pos));
    ll_store(bcast + 2, c.tag, static_cast<unsigned>(o.n));
    ll_store(bcast + 3, c.tag, stop ? 1u : 0u);
    tl.mark(kTlLm + kTlFinStored);
    // the token to the host as well (the host polls for it; the token is the whole message, so no
    // ordering with other stores is needed)
    if (H.host_tokens && n_tok < a.max_pos)
      __hip_atomic_store(H.host_tokens + n_tok, o.tok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    s.warm[0] = o.tok;
    s.warm[1] = o.pos;
  }
  if (FW_EMBED_WARM && NV == 1) {
    // The next step's embedding and position rows, read here with cached loads once the token is
    // broadcast: the layer-0 LayerNorm blocks, which read them about a microsecond later, then find
    // them in the memory-side cache instead of HBM. This block's first phase of the next step comes
    // later, so the wait for the loads is off the step's path.
    __syncthreads();
    const _Float16 *ea, *eb;
    embed_rows_of(s.warm[0], s.warm[1], a.embed, a.pos_embed, a.vocab, a.max_pos, &ea, &eb);
    if (tid < 2 * (kHidden / 8)) {
      const uint4 v = reinterpret_cast<const uint4*>(tid < kHidden / 8 ? ea : eb)[tid % (kHidden / 8)];
      asm volatile("" ::"v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w));
    }
  }
}

// ---------------------------------------------------------------------------------------------
// The kernel
// ---------------------------------------------------------------------------------------------
struct Sched {
  int start;  // first block of the current phase's run
  int G;
  __device__ int rank() const { return (static_cast<int>(blockIdx.x) - start + G) % G; }
  __device__ void next(int used) { start = (start + used) % G; }
};

// The kernel's arguments, re-read from the kernel-argument segment wherever this is called: the
// pointer is opaque to the compiler, so it cannot hoist argument loads out of the step loop and keep
// them in registers across a whole step (scalar loads of the segment are cheap; the registers are not).
// The area from the kernel arguments directly (not through step_args: the compiler may keep the address
// in two scalar registers across the launch, which every hand-off uses).
__device__ __forceinline__ const uint64_t* step_area() {
  return hx_area(((const StepArgs*)__builtin_amdgcn_kernarg_segment_ptr())->ws);  // an address-space cast
}

__device__ __forceinline__ const StepArgs& step_args() {
  auto p = __builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(p));
  return *(const StepArgs*)p;  // the constant-segment pointer as a generic one (an address-space cast)
}

// NV = 1: n_steps decoder steps. NV = kPromptLen: the prompt pass, one step over NV positions at once
// (every phase on NV vectors; the LM head on the last).
template <int NV>
__global__ void __launch_bounds__(kStepThreads) decoder_step_kernel(StepArgs args) {
  const StepArgs& a = args;
  __shared__ __align__(16) _Float16 h_res[NV * kHidden];
  __shared__ __align__(16) _Float16 x_lds[NV * kStepFfn];  // also the self attention's wave partials
  static_assert(sizeof(x_lds) >= (2 + kHeadDim) * kMaxCombineSplits * 4 * sizeof(float), "self-attention slots");
  __shared__ __align__(16) uint4 kvf[NV > 1 ? NV : 1][2][8];  // the prompt pass: fresh k / v rows of a head
  __shared__ float red[8 * kStepWaves];  // LayerNorm sums (16 slots each for the LM head's 1024-thread order)
  __shared__ __align__(16) LmLds lm;
  __shared__ float wgt[kMaxCombineHeads * kMaxCombineSplits];
  __shared__ float den[kMaxCombineHeads];
  __shared__ AttnLds att;
  __shared__ std::conditional_t<(NV > 1), AttnNvLds<NV>, char> attv;  // the prompt pass's cross attention
  __shared__ float part_lds[kMaxCombineSplits * kPartWords];
  __shared__ unsigned epoch_lds;
  __shared__ unsigned bcast_lds[4];
  __shared__ unsigned stage[NV * kMaxPasses * kStepWaves];  // a GEMV phase's output words before their coalesced store
  const int tid = threadIdx.x, wave = tid >> 6;
  const int G = gridDim.x;
  unsigned* ctl = reinterpret_cast<unsigned*>(a.ws);
  uint64_t* regions = const_cast<uint64_t*>(step_area());  // the logical layout's base
  const int xcc = xcc_id();
  for (int i = tid; i < kMaxPages / 32; i += kStepThreads)
    hx_groups[i] = reinterpret_cast<const unsigned*>(a.ws + kCtlBytes)[i];  // read after the barrier below

  // The launch's tags: the epoch every block reads before it arrives; step st of the launch tags its
  // words epoch + 1 + st. The last block to arrive moves the epoch on by the launch's steps, when no
  // block of this one can still be reading it.
  Tl::clear();
  if (tid == 0) epoch_lds = __hip_atomic_load(ctl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const unsigned epoch = epoch_lds;
  unsigned arrived = 0;
  if (tid == 0) arrived = atomicAdd(ctl + 1, 1u);
  uint64_t* maxima = regions + static_cast<size_t>(a.n_layers) * NV * kLayerWords;
  uint64_t* bcast = maxima + 2 * kMaxGrid;

  if (a.has_head)
    for (int i = tid; i < kHidden / 2; i += kStepThreads) {
      lm.gamma[i] = reinterpret_cast<const h2v*>(a.head.gamma)[i];
      lm.beta[i] = reinterpret_cast<const h2v*>(a.head.beta)[i];
    }
  StepPos sp{a.cur[0], a.state[0]};
  int64_t n_tok = a.has_head && blockIdx.x == fin_block() ? a.state[1] : 0;  // for the finalize
  const int ns_cross = (a.enc_len + kCrossSplitKeys - 1) / kCrossSplitKeys;

  // Runs of blocks per phase (step_workers), taken in turn around the grid: consecutive phases use
  // disjoint blocks, and the LN3 + fc1 phase reuses only the first half of the cross-attention run
  // (its blocks finish their items early; the blocks that combine a head's splits are the run's last).
  // Every step starts the runs at block 0, so a layer's phase
  // runs on the same blocks in every step: the self-attention block of a head reads back the cache
  // rows it wrote itself (through its own CU's caches) in the steps before.
  const StepWorkers wk = step_workers(G);
  const int w_vec = wk.vec, w_cross = wk.cross, w_qkv = wk.qkv, w_fc1 = wk.fc1;
  // the resident LM-head rows (the decode steps only: the prompt pass's vectors fill that LDS)
  if (NV == 1 && a.has_head && a.lm_res_rows > 0) {  // the share's last rows, once for every step of the launch
    const LmResView res = lm_res_view(a.lm_res_rows);
    const LmShare share = lm_share(a.vocab, a.n_layers);
    const int n_res = min(res.rows, share.r1 - share.r0), rb = share.r1 - n_res;
    const uint4* src = reinterpret_cast<const uint4*>(a.head.wq) + static_cast<size_t>(rb) * kQ8Chunks;
    for (int i = tid; i < n_res * kQ8Chunks; i += kStepThreads) lm_res_lds[i] = ld_lm_head(src + i);
    for (int i = tid; i < n_res; i += kStepThreads) {
      const_cast<float2*>(res.meta)[i] = a.head.meta[rb + i];
      const_cast<uint8_t*>(res.sup)[i] = a.head.suppress[rb + i];
    }  // read after the barriers of the first step's phases
  }

  const int n_steps = NV > 1 ? 1 : args.n_steps;
  for (int st = 0; st < n_steps; ++st) {
    const StepArgs& a = step_args();
    const Ll c{ctl, epoch + 1u + static_cast<unsigned>(st), a.spin_limit, xcc};
    const Tl tl = Tl::at(st);
    constexpr int kBcastWave = kStepWaves - 1;  // polls the previous step's token
    // Layer 0's q/k/v rows do not depend on the token: the blocks of that run (it starts at block 0) read
    // them into their XCD's L2 while they wait for it, so the phase finds them there. The wave that polls
    // for the token reads none (its poll would return behind them), and the others take the loads' values
    // only after the token is in (a wait for them before the barrier would hold the poll back).
    Gv<kHidden, 2> gw;
    const bool warm = FW_QKV_WARM && NV == 1 && st > 0 && static_cast<int>(blockIdx.x) < w_qkv && wave != kBcastWave;
    if (warm)
      gv_load(gw, a.layer[0].qkv_w, a.layer[0].qkv_b, kQkvWords, static_cast<int>(blockIdx.x) * kStepWaves + wave,
              w_qkv * kStepWaves);
    if (st > 0) {  // the previous step's token, position, token count and stop flag
      __syncthreads();
      const int bt = tid - kBcastWave * kWave;
      if (bt >= 0 && bt < 4) {
        const int idx[1] = {bt};
        unsigned v[1];
        const Ll prev{ctl, c.tag - 1u, a.spin_limit, xcc};
        ll_wait<1>(bcast, idx, v, prev);
        bcast_lds[bt] = v[0];
      }
      __syncthreads();
      sp.tok = __builtin_amdgcn_readfirstlane(bcast_lds[0]);  // uniform: scalar registers
      sp.pos_raw = static_cast<int>(__builtin_amdgcn_readfirstlane(bcast_lds[1]));
      n_tok = static_cast<int>(__builtin_amdgcn_readfirstlane(bcast_lds[2]));
      if (__builtin_amdgcn_readfirstlane(bcast_lds[3])) break;  // an end-of-text token: every block stops
    }
    if (warm) {
      unsigned x = 0;
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int k = 0; k < Gv<kHidden, 2>::RS::kC; ++k) x ^= gw.w[u][0][k].x;
      asm volatile("" ::"v"(x));  // the loads complete by here, not in the phase
    }
    tl.mark(0);
    tl.mark_shader_clock(kTlClk + kTlClkStart);
    const int pos = static_cast<int>(sp.pos_raw < 0 ? 0 : (sp.pos_raw >= a.max_pos ? a.max_pos - 1 : sp.pos_raw));
    const int ns_self = (pos + kSelfSplitKeys) / kSelfSplitKeys;
    Sched sc{0, G};
    int applied = 0;  // residual contributions added to h_res

    for (int l = 0; l < a.n_layers; ++l) {
      const StepLayer& L = a.layer[l];
      uint64_t* R = regions + static_cast<size_t>(l) * NV * kLayerWords;

      // 1: residual + LN1 + q/k/v (1920 pairs)
      {
        __syncthreads();
        const int rank = sc.rank(), W = w_qkv;
        constexpr int U = 2;
        const int npairs = kQkvWords;
        if (rank < W) {
          Gv<kHidden, U> g;
          int base = rank * kStepWaves;  // the block's first word; a block-uniform loop over passes of U words
          const int qs = W * kStepWaves;
          EmbRegs emb;
          const bool emb_first = NV == 1 && applied == 0;  // block-uniform: layer 0 of a step
          if (emb_first) embed_load(emb, a, sp);
          gv_load(g, L.qkv_w, L.qkv_b, npairs, base + wave, qs);
          LnRegs<kStepThreads> lnr;
          ln_params(lnr, L.ln1_g, L.ln1_b);
          if (emb_first) embed_store(emb, h_res, applied);
          tl.phase(l, 1, 0);
          resid_catch_up<kStepThreads, NV>(h_res, applied, 1 + 3 * l, regions, a, c, sp);
          tl.phase(l, 1, 3);
          resid_layernorm_nv<NV>(lnr, h_res, L.eps1, x_lds, red);
          __syncthreads();
          tl.phase(l, 1, 1);
          for (;;) {
            gv_finish_nv<kHidden, U, FW_ACT_NONE, NV>(g, x_lds, stage, R + NV * kOffQkv, c.tag, base, qs, npairs);
            base += U * qs;
            if (base >= npairs) break;
            __syncthreads();
            gv_load(g, L.qkv_w, L.qkv_b, npairs, base + wave, qs);
          }
          tl.phase(l, 1, 2);
        }
        sc.next(W);
      }
      // 2: self attention, one block per head (its splits combined in the block)
      {
        __syncthreads();
        const int rank = sc.rank(), W = kStepHeads * NV;  // (head, vector) pairs
        if (rank < W) {
          const int z = rank / kStepHeads;
          tl.phase(l, 2, 0);
          self_attn_head<NV>(c, rank % kStepHeads, z,
                             NV > 1 ? (min(pos + z, a.max_pos - 1) + kSelfSplitKeys) / kSelfSplitKeys : ns_self,
                             L.self_k, L.self_v, a.max_pos, pos, R + NV * kOffQkv, R + NV * kOffSelfVec, a.scale, att,
                             part_lds, reinterpret_cast<float*>(x_lds), kvf, tl,
                             l < kTlLayers ? tl_phase(l, 2) : kTlSlots - 4);
          tl.phase(l, 2, 2);
        }
        sc.next(w_qkv);
      }
      // 3: out projection (640 pairs)
      {
        __syncthreads();
        const int rank = sc.rank(), W = w_vec;
        constexpr int U = 1;
        const int npairs = kVecWords;
        if (rank < W) {
          Gv<kHidden, U> g;
          int base = rank * kStepWaves;  // the block's first word; a block-uniform loop over passes of U words
          const int qs = W * kStepWaves;
          gv_load(g, L.out_w, L.out_b, npairs, base + wave, qs);
          tl.phase(l, 3, 0);
          if (FW_EAGER_CATCH_UP) resid_catch_up<kStepThreads, NV>(h_res, applied, 1 + 3 * l, regions, a, c, sp);
          fetch_attn_vectors<NV>(R + NV * kOffSelfVec, x_lds, c);
          __syncthreads();
          tl.phase(l, 3, 1);
          for (;;) {
            gv_finish_nv<kHidden, U, FW_ACT_NONE, NV>(g, x_lds, stage, R + NV * kOffAttnOut, c.tag, base, qs, npairs);
            base += U * qs;
            if (base >= npairs) break;
            __syncthreads();
            gv_load(g, L.out_w, L.out_b, npairs, base + wave, qs);
          }
          tl.phase(l, 3, 2);
        }
        sc.next(W);
      }
      // 4: residual + LN2 + cross q (640 pairs)
      {
        __syncthreads();
        const int rank = sc.rank(), W = w_vec;
        constexpr int U = 1;
        const int npairs = kVecWords;
        if (rank < W) {
          Gv<kHidden, U> g;
          int base = rank * kStepWaves;  // the block's first word; a block-uniform loop over passes of U words
          const int qs = W * kStepWaves;
          gv_load(g, L.cq_w, L.cq_b, npairs, base + wave, qs);
          LnRegs<kStepThreads> lnr;
          ln_params(lnr, L.ln2_g, L.ln2_b);
          tl.phase(l, 4, 0);
          resid_catch_up<kStepThreads, NV>(h_res, applied, 2 + 3 * l, regions, a, c, sp);
          tl.phase(l, 4, 3);
          resid_layernorm_nv<NV>(lnr, h_res, L.eps2, x_lds, red);
          __syncthreads();
          tl.phase(l, 4, 1);
          for (;;) {
            gv_finish_nv<kHidden, U, FW_ACT_NONE, NV>(g, x_lds, stage, R + NV * kOffCrossQ, c.tag, base, qs, npairs);
            base += U * qs;
            if (base >= npairs) break;
            __syncthreads();
            gv_load(g, L.cq_w, L.cq_b, npairs, base + wave, qs);
          }
          tl.phase(l, 4, 2);
        }
        sc.next(W);
      }
      // 5: cross-attention splits, each head combined by the block that ran its last split
      {
        __syncthreads();
        const int nitems = kStepHeads * ns_cross;  // (head, split) items; each runs the NV queries
        const int rank = sc.rank();
        if constexpr (NV == 1) {
          const int W = min(w_cross, nitems);
          if (rank < W) {
            tl.phase(l, 5, 0);
            cross_attn_items(c, rank, W, ns_cross, L.cross_k, L.cross_v, a.enc_len, R + kOffCrossQ, R + kOffCrossPart,
                             R + kOffCrossVec, a.scale, att, part_lds, tl, l < kTlLayers ? tl_phase(l, 5) : kTlSlots - 4);
          }
        } else {  // two items per block on the second half of the run (LN3 + fc1 reuses the first half)
          const int lo = w_cross / 2, W = min(w_cross - lo, (nitems + 1) / 2);
          if (rank >= lo && rank - lo < W)
            cross_attn_items_nv<NV>(c, rank - lo, W, nitems, ns_cross, L.cross_k, L.cross_v, a.enc_len,
                                    R + NV * kOffCrossQ, R + NV * kOffCrossPart, R + NV * kOffCrossVec, a.scale, attv,
                                    part_lds, wgt, den);
        }
        sc.next(w_cross);
      }
      // 6: cross-out projection (640 pairs)
      {
        __syncthreads();
        const int rank = sc.rank(), W = w_vec;
        constexpr int U = 1;
        const int npairs = kVecWords;
        if (rank < W) {
          Gv<kHidden, U> g;
          int base = rank * kStepWaves;  // the block's first word; a block-uniform loop over passes of U words
          const int qs = W * kStepWaves;
          gv_load(g, L.co_w, L.co_b, npairs, base + wave, qs);
          tl.phase(l, 6, 0);
          if (FW_EAGER_CATCH_UP) resid_catch_up<kStepThreads, NV>(h_res, applied, 2 + 3 * l, regions, a, c, sp);
          fetch_attn_vectors<NV>(R + NV * kOffCrossVec, x_lds, c);
          __syncthreads();
          tl.phase(l, 6, 1);
          for (;;) {
            gv_finish_nv<kHidden, U, FW_ACT_NONE, NV>(g, x_lds, stage, R + NV * kOffCrossOut, c.tag, base, qs, npairs);
            base += U * qs;
            if (base >= npairs) break;
            __syncthreads();
            gv_load(g, L.co_w, L.co_b, npairs, base + wave, qs);
          }
          tl.phase(l, 6, 2);
        }
        sc.next(W);
      }
      // 7: residual + LN3 + fc1 + GELU (2560 pairs)
      {
        __syncthreads();
        const int rank = sc.rank(), W = w_fc1;
        constexpr int U = 3;
        const int npairs = kFfnWords;
        if (rank < W) {
          Gv<kHidden, U> g;
          int base = rank * kStepWaves;  // the block's first word; a block-uniform loop over passes of U words
          const int qs = W * kStepWaves;
          gv_load(g, L.fc1_w, L.fc1_b, npairs, base + wave, qs);
          LnRegs<kStepThreads> lnr;
          ln_params(lnr, L.ln3_g, L.ln3_b);
          tl.phase(l, 7, 0);
          resid_catch_up<kStepThreads, NV>(h_res, applied, 3 + 3 * l, regions, a, c, sp);
          tl.phase(l, 7, 3);
          resid_layernorm_nv<NV>(lnr, h_res, L.eps3, x_lds, red);
          __syncthreads();
          tl.phase(l, 7, 1);
          for (;;) {
            gv_finish_nv<kHidden, U, FW_ACT_GELU, NV>(g, x_lds, stage, R + NV * kOffFfn, c.tag, base, qs, npairs);
            base += U * qs;
            if (base >= npairs) break;
            __syncthreads();
            gv_load(g, L.fc1_w, L.fc1_b, npairs, base + wave, qs);
          }
          tl.phase(l, 7, 2);
        }
        sc.next(W);
      }
      // 8: fc2 (640 pairs of 5120-wide rows)
      {
        __syncthreads();
        const int rank = sc.rank(), W = w_vec;
        constexpr int U = 1;
        const int npairs = kVecWords;
        const bool last = l + 1 == a.n_layers;
        if (rank < W) {
          Gv<kStepFfn, U> g;
          int base = rank * kStepWaves;  // the block's first word; a block-uniform loop over passes of U words
          const int qs = W * kStepWaves;
          gv_load(g, L.fc2_w, L.fc2_b, npairs, base + wave, qs);
          tl.phase(l, 8, 0);
          if (FW_EAGER_CATCH_UP) resid_catch_up<kStepThreads, NV>(h_res, applied, 3 + 3 * l, regions, a, c, sp);
          // the fc1 output, 2560 words per vector, into LDS
          constexpr int kPer = kFfnWords / kStepThreads;
          static_assert(kFfnWords % kStepThreads == 0, "whole words per thread");
          for (int vec = 0; vec < NV; ++vec) {
            int idx[kPer];
#pragma unroll
            for (int k = 0; k < kPer; ++k) idx[k] = tid + k * kStepThreads;
            unsigned v[kPer];
            ll_wait<kPer>(R + NV * kOffFfn + vec * kFfnWords, idx, v, c);
#pragma unroll
            for (int k = 0; k < kPer; ++k) reinterpret_cast<unsigned*>(x_lds + vec * kStepFfn)[idx[k]] = v[k];
          }
          __syncthreads();
          tl.phase(l, 8, 1);
          for (;;) {
            if constexpr (NV == 1)
              gv_finish<kStepFfn, U, FW_ACT_NONE>(g, x_lds, stage, R + kOffMlpOut, c.tag, last ? a.x_out : nullptr, base,
                                                  qs, npairs);
            else
              gv_finish_nv<kStepFfn, U, FW_ACT_NONE, NV>(g, x_lds, stage, R + NV * kOffMlpOut, c.tag, base, qs, npairs);
            base += U * qs;
            if (base >= npairs) break;
            __syncthreads();
            gv_load(g, L.fc2_w, L.fc2_b, npairs, base + wave, qs);
          }
          tl.phase(l, 8, 2);
        }
        sc.next(W);
      }
    }

    if (a.has_head) {
      __syncthreads();
      lm_head_phase<NV>(a, a.head, c, h_res, applied, regions, maxima, bcast, x_lds, red, lm, sp, n_tok, tl);
    } else if (NV == 1 && blockIdx.x == 0) {
      // the residual the LM head adds the last fc2 output to: everything up to the last cross-out
      __syncthreads();
      resid_catch_up(h_res, applied, 3 * a.n_layers, regions, a, c, sp);  // the last fc2 output stays out
      __syncthreads();
      for (int i = tid; i < kHidden / 2; i += kStepThreads)
        reinterpret_cast<unsigned*>(a.h_out)[i] = reinterpret_cast<const unsigned*>(h_res)[i];
    }
    if (FW_STEP_TIMELINE) {
      tl.mark_shader_clock(kTlClk + kTlClkEnd);
      tl.mark(kTlClk + kTlClkWallEnd);
      __syncthreads();
      tl.flush();
    }
  }
  if (tid == 0 && arrived == static_cast<unsigned>(G) - 1u) {
    __hip_atomic_store(ctl + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(ctl, epoch + static_cast<unsigned>(n_steps), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Which half of the chip the first physical page of each logical page of the hand-off area is local to
// (the group's other pages alternate from it). The blocks on XCDs 0 and 1 (half 0) hand a word of that
// page back and forth kCalIters times, as do the blocks on XCDs 4 and 5 (half 1) on another line of the
// page; a page is local to the pair that does it faster (about 0.4 against 0.6 us a hand-off). step_calibrate_clear first zeroes the words used (and the latencies), and
// step_calibrate_finish turns the latencies into the group bits and zeroes the words again. Every wait is
// bounded: a pair whose partner does not run (another XCD numbering) stops and leaves its latencies 0,
// and its pages keep bit 0 (each copy of a word then sits on a fixed page of the pair: correct, only not
// placed by locality).
constexpr int kCalIters = 16;
constexpr int kCalWord[2] = {8, 8 + kPageWords / 2};  // one 128-byte line per pair, in the page's halves
constexpr int kCalClaim = 16;   // control words 16-23: one claim per XCD (the first block there takes it)
constexpr int kCalDone = 3;     // control word 3: pages calibrated by both pairs (the last calibration)
__global__ void __launch_bounds__(256) step_calibrate_clear(unsigned char* ws, int n_pages) {
  uint64_t* area = hx_area(ws);
  float* lat = reinterpret_cast<float*>(ws + kCtlBytes + kGroupBytes);
  unsigned* ctl = reinterpret_cast<unsigned*>(ws);
  if (threadIdx.x < 8) ctl[kCalClaim + threadIdx.x] = 0u;
  if (threadIdx.x == 0) ctl[kCalDone] = 0u;
  for (int j = threadIdx.x; j < n_pages; j += blockDim.x) {
    area[static_cast<size_t>(j) * kCopies * kPageWords + kCalWord[0]] = 0;
    area[static_cast<size_t>(j) * kCopies * kPageWords + kCalWord[1]] = 0;
    lat[j] = 0.f;
    lat[kMaxPages + j] = 0.f;
  }
}
__global__ void __launch_bounds__(64) step_calibrate_kernel(unsigned char* ws, int n_pages) {
  if (threadIdx.x != 0) return;
  unsigned xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  xcc &= 0xf;
  const int pair = (xcc == 0 || xcc == 1) ? 0 : ((xcc == 4 || xcc == 5) ? 1 : -1);
  unsigned* ctl = reinterpret_cast<unsigned*>(ws);
  // one block per role: the first of the launch's blocks to land on the XCD (the launch has 8 per XCD)
  if (pair < 0 || atomicCAS(ctl + kCalClaim + xcc, 0u, 1u) != 0u) return;
  const int me = static_cast<int>(xcc & 1);
  uint64_t* area = hx_area(ws);
  float* lat = reinterpret_cast<float*>(ws + kCtlBytes + kGroupBytes) + pair * kMaxPages;
  constexpr long long kLimit = 200000;  // 2 ms of the 100 MHz clock per wait
  auto wait_for = [&](const uint64_t* w, uint64_t v) {
    const long long t0 = wall_clock64();
    for (int it = 1; __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < v; ++it)
      if ((it & 15) == 0 && wall_clock64() - t0 > kLimit) return false;
    return true;
  };
  for (int j = 0; j < n_pages; ++j) {
    uint64_t* w = area + static_cast<size_t>(j) * kCopies * kPageWords + kCalWord[pair];
    const long long t0 = wall_clock64();
    for (int i = 1; i <= kCalIters; ++i) {  // block 0 of the pair stores odd values, block 1 even ones
      if ((me == 1 || i > 1) && !wait_for(w, 2ull * i - (me == 0 ? 2 : 1))) return;
      __hip_atomic_store(w, 2ull * i - (me == 0 ? 1 : 0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!wait_for(w, 2ull * kCalIters)) return;
    if (me == 0) lat[j] = static_cast<float>(wall_clock64() - t0);
  }
  if (me == 0) atomicAdd(ctl + kCalDone, 1u);  // 2 once both pairs have measured every page
}
__global__ void __launch_bounds__(256) step_calibrate_finish(unsigned char* ws, int n_pages) {
  uint64_t* area = hx_area(ws);
  const float* lat = reinterpret_cast<const float*>(ws + kCtlBytes + kGroupBytes);
  unsigned* groups = reinterpret_cast<unsigned*>(ws + kCtlBytes);
  for (int i = threadIdx.x; i < kMaxPages / 32; i += blockDim.x) {
    unsigned bits = 0;
    for (int b = 0; b < 32; ++b) {
      const int j = i * 32 + b;
      if (j < n_pages && lat[j] > 0.f && lat[kMaxPages + j] > 0.f && lat[kMaxPages + j] < lat[j]) bits |= 1u << b;
    }
    groups[i] = bits;
  }
  for (int j = threadIdx.x; j < n_pages; j += blockDim.x) {
    area[static_cast<size_t>(j) * kCopies * kPageWords + kCalWord[0]] = 0;
    area[static_cast<size_t>(j) * kCopies * kPageWords + kCalWord[1]] = 0;
  }
}

}  // namespace
}  // namespace fw

using namespace fw;

static size_t step_logical_pages(int n_layers);

extern "C" int fw_decoder_step_calibrate(void* workspace, int64_t ws_bytes, int n_layers, hipStream_t stream) {
  const size_t need = fw_decoder_step_workspace_bytes(n_layers);
  if (!workspace || need == 0 || ws_bytes < static_cast<int64_t>(need))
    return fw_fail(FW_EINVAL, "decoder_step_calibrate: workspace of %lld bytes, %zu needed for %d layers",
                   static_cast<long long>(ws_bytes), need, n_layers);
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  const int n_pages = static_cast<int>(step_logical_pages(n_layers));  // the first page of each group
  hipLaunchKernelGGL(step_calibrate_clear, dim3(1), dim3(256), 0, stream, ws, n_pages);
  hipLaunchKernelGGL(step_calibrate_kernel, dim3(64), dim3(64), 0, stream, ws, n_pages);
  hipLaunchKernelGGL(step_calibrate_finish, dim3(1), dim3(256), 0, stream, ws, n_pages);
  return fw_check_launch("decoder_step_calibrate");
}

extern "C" int fw_decoder_step_calibrated(const void* workspace) {
  unsigned v = 0;
  if (!workspace || hipMemcpy(&v, static_cast<const unsigned*>(workspace) + kCalDone, sizeof(v), hipMemcpyDeviceToHost) != hipSuccess)
    return fw_fail(FW_EHIP, "decoder_step_calibrated: cannot read the workspace");
  return v == 2u ? 1 : 0;
}

extern "C" void* fw_host_alloc_coherent(size_t bytes) {
  void* p = nullptr;
  if (bytes == 0 || hipHostMalloc(&p, bytes, hipHostMallocCoherent) != hipSuccess) {
    fw_fail(FW_EHIP, "host_alloc_coherent: hipHostMalloc of %zu bytes failed", bytes);
    return nullptr;
  }
  return p;
}

extern "C" void fw_host_free(void* p) {
  if (p) (void)hipHostFree(p);
}

// Logical pages of the hand-off regions: each layer's regions (for the prompt pass's kPromptLen vectors),
// the LM head's block maxima and the token broadcast.
static size_t step_logical_pages(int n_layers) {
  const size_t words = static_cast<size_t>(n_layers) * kPromptLen * kLayerWords + 2 * kMaxGrid + 8;
  return (words + kPageWords - 1) / kPageWords;
}
static_assert((static_cast<size_t>(kStepMaxLayers) * kPromptLen * kLayerWords + 2 * kMaxGrid + 8 + kPageWords - 1) /
                  kPageWords <= kMaxPages,
              "one group bit per logical page");

extern "C" size_t fw_decoder_step_workspace_bytes(int n_layers) {
  if (n_layers < 1 || n_layers > kStepMaxLayers) return 0;
  // control words, each layer's hand-off regions (for the prompt pass's kPromptLen vectors), the LM
  // head's per-block maxima, then the words the finalizing block broadcasts to the next step (four, in
  // eight)
  const size_t pages = step_logical_pages(n_layers);
  return kCtlBytes + kGroupBytes + kCalibBytes + kAreaAlign + kCopies * pages * kPageWords * sizeof(uint64_t);
}

extern "C" int fw_decoder_step_max_layers(void) { return kStepMaxLayers; }

// LM-head rows per block that fit in the step kernel's dynamic LDS on the current device (cached per
// device): the device's LDS per block less the kernel's static LDS, at most kLmResRows.
static int step_resident_rows(int dev) {
  constexpr int kDevs = 64;
  static int cached[kDevs];  // rows + 1, 0 = not yet computed (a race computes the same value twice)
  if (dev >= 0 && dev < kDevs && cached[dev] > 0) return cached[dev] - 1;
  int max_lds = 0;
  hipFuncAttributes fa{};
  int rows = 0;
  if (hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess &&
      hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(decoder_step_kernel<1>)) == hipSuccess &&
      static_cast<size_t>(max_lds) > fa.sharedSizeBytes) {
    const size_t avail = static_cast<size_t>(max_lds) - fa.sharedSizeBytes;
    rows = kLmResRows;
    while (rows > 0 && lm_res_bytes(rows) > avail) rows -= 4;
    if (rows > 0 && hipFuncSetAttribute(reinterpret_cast<const void*>(decoder_step_kernel<1>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        static_cast<int>(lm_res_bytes(rows))) != hipSuccess)
      rows = 0;
  }
  (void)hipGetLastError();  // a failed query leaves no error for the launch check: the rows are then 0
  if (dev >= 0 && dev < kDevs) cached[dev] = rows + 1;
  return rows;
}

extern "C" int fw_decoder_step_timeline_slots(void) { return FW_STEP_TIMELINE ? kTlSlots : 0; }

extern "C" int fw_decoder_step_timeline(void* buf, int64_t bytes, int steps) {
#if FW_STEP_TIMELINE
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return fw_fail(FW_EHIP, "decoder_step_timeline: cannot read the device's CU count");
  const int grid = cus < kMaxGrid ? cus : kMaxGrid;
  if (buf && (steps < 1 || bytes < static_cast<int64_t>(steps) * grid * kTlSlots * 8))
    return fw_fail(FW_EINVAL, "decoder_step_timeline: %lld bytes do not hold %d steps of %d blocks x %d slots",
                   static_cast<long long>(bytes), steps, grid, kTlSlots);
  long long* p = static_cast<long long*>(buf);
  const int n = buf ? steps : 0;
  if (hipMemcpyToSymbol(HIP_SYMBOL(g_step_tl), &p, sizeof(p)) != hipSuccess ||
      hipMemcpyToSymbol(HIP_SYMBOL(g_step_tl_steps), &n, sizeof(n)) != hipSuccess)
    return fw_fail(FW_EHIP, "decoder_step_timeline: hipMemcpyToSymbol failed");
  return FW_OK;
#else
  (void)buf, (void)bytes, (void)steps;
  return fw_fail(FW_EINVAL, "decoder_step_timeline: this library was built without FW_STEP_TIMELINE");
#endif
}

extern "C" int fw_decoder_step_resident_rows(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fw_fail(FW_EHIP, "decoder_step_resident_rows: no device");
  return step_resident_rows(dev);
}

// The sizes a launch takes, checked against the device: the grid is the CU count (at most kMaxGrid), and
// every phase must find its blocks in it (the self attention's one block per head and vector within the
// run after the q/k/v run; the LM head's largest share within the candidate list). Returns FW_OK and the
// grid, or FW_EINVAL / FW_EHIP with the reason.
static int step_range_check(const char* name, int n_layers, int vocab, int max_pos, int enc_len) {
  if (n_layers < 1 || n_layers > kStepMaxLayers)
    return fw_fail(FW_EINVAL, "%s: n_layers must be in [1, %d]", name, kStepMaxLayers);
  if (vocab < 1 || max_pos < 1 || max_pos > kMaxCombineSplits * kSelfSplitKeys)
    return fw_fail(FW_EINVAL, "%s: max_pos must be in [1, %d]", name, kMaxCombineSplits * kSelfSplitKeys);
  if (enc_len < 1 || enc_len > kMaxCombineSplits * kCrossSplitKeys)
    return fw_fail(FW_EINVAL, "%s: enc_len must be in [1, %d]", name, kMaxCombineSplits * kCrossSplitKeys);
  return FW_OK;
}

static int step_sizes_check(const char* name, int n_layers, int vocab, int max_pos, int enc_len, bool has_head,
                            int nv, int* grid_out) {
  if (const int st = step_range_check(name, n_layers, vocab, max_pos, enc_len)) return st;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus < 1)
    return fw_fail(FW_EHIP, "%s: cannot read the device's CU count", name);
  const int grid = cus < kMaxGrid ? cus : kMaxGrid;
  const int w_vec = std::min(kVecWorkers, std::max(1, grid * 5 / 16));
  if (grid - w_vec < kStepHeads * nv)  // the self attention: a block per (head, vector) in the run after q/k/v
    return fw_fail(FW_EINVAL, "%s: %d CUs run too few blocks (the self attention needs %d beside %d others)", name,
                   grid, kStepHeads * nv, w_vec);
  if (has_head) {
    // the largest share (any placement of the late run)
    int most = 0;
    for (int b = 0; b < grid; ++b)
      most = std::max(most, lm_rows_before(b + 1, vocab, grid, 0, w_vec) - lm_rows_before(b, vocab, grid, 0, w_vec));
    if (most + 1 > kLmMaxBatches * kLmBatchRows)  // + 1: the rounding of another placement of the late run
      return fw_fail(FW_EINVAL, "%s: vocab %d gives a block %d rows of the LM head (at most %d) on %d blocks", name,
                     vocab, most, kLmMaxBatches * kLmBatchRows, grid);
  }
  *grid_out = grid;
  return FW_OK;
}

extern "C" int fw_decoder_step_check(int n_layers, int vocab, int max_pos, int enc_len, int prompt) {
  int grid = 0;
  return step_sizes_check("decoder_step_check", n_layers, vocab, max_pos, enc_len, true, prompt ? kPromptLen : 1,
                          &grid);
}

static int decoder_step_launch(const char* name, const fw_dec_layer* layers, int n_layers, const fw_dec_head* head,
                               const int64_t* prompt, int n_steps, int64_t* cur, int64_t* state, const void* embed, const void* pos_embed, int vocab,
                               int max_pos, int enc_len, float scale, void* h_out, void* x_out, void* workspace,
                               int64_t ws_bytes, int64_t spin_limit, hipStream_t stream) {
  if (!layers || !cur || !state || !embed || !pos_embed || !workspace || (!head && (!h_out || !x_out)))
    return fw_fail(FW_EINVAL, "%s: null pointer", name);
  if (n_steps < 1 || n_steps > kStepMaxSteps || (!head && n_steps != 1))
    return fw_fail(FW_EINVAL, "%s: n_steps must be in [1, %d] (1 without the LM head)", name, kStepMaxSteps);
  if (prompt && (!head || n_steps != 1)) return fw_fail(FW_EINVAL, "%s: the prompt pass is one step with the LM head", name);
  if (const int st = step_range_check(name, n_layers, vocab, max_pos, enc_len)) return st;
  if (ws_bytes < static_cast<int64_t>(fw_decoder_step_workspace_bytes(n_layers)))
    return fw_fail(FW_EINVAL, "%s: workspace too small (%lld < %zu bytes)", name, static_cast<long long>(ws_bytes),
                   fw_decoder_step_workspace_bytes(n_layers));
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) || (reinterpret_cast<uintptr_t>(h_out) & 3u) ||
      (reinterpret_cast<uintptr_t>(x_out) & 3u))
    return fw_fail(FW_EINVAL, "%s: workspace must be 256-byte and h_out / x_out 4-byte aligned", name);
  if (spin_limit < 0) return fw_fail(FW_EINVAL, "%s: spin_limit must be >= 0", name);
  if (head) {
    const fw_dec_head& hd = *head;
    if (!hd.ln_gamma || !hd.ln_beta || !hd.w || !hd.wq || !hd.meta || !hd.suppress || !hd.tokens)
      return fw_fail(FW_EINVAL, "%s: null LM-head tensor", name);
    if ((reinterpret_cast<uintptr_t>(hd.w) & 15u) || (reinterpret_cast<uintptr_t>(hd.wq) & 15u) ||
        (reinterpret_cast<uintptr_t>(hd.meta) & 7u) || (reinterpret_cast<uintptr_t>(hd.y_out) & 3u) ||
        (reinterpret_cast<uintptr_t>(hd.host_tokens) & 7u))
      return fw_fail(FW_EINVAL, "%s: w and wq must be 16-byte aligned, meta and host_tokens 8-byte and y_out 4-byte aligned",
                     name);
    if (hd.n_eos < 0 || hd.n_eos > kStepMaxEos)
      return fw_fail(FW_EINVAL, "%s: n_eos must be in [0, %d]", name, kStepMaxEos);
  }
  StepArgs a{};
  for (int l = 0; l < n_layers; ++l) {
    const fw_dec_layer& s = layers[l];
    const void* must[] = {s.ln1_gamma, s.ln1_beta, s.qkv_w, s.out_w, s.ln2_gamma, s.ln2_beta, s.cross_q_w,
                          s.cross_out_w, s.ln3_gamma, s.ln3_beta, s.fc1_w, s.fc2_w, s.self_k, s.self_v,
                          s.cross_k, s.cross_v};
    for (const void* p : must)
      if (!p) return fw_fail(FW_EINVAL, "%s: layer %d has a null tensor", name, l);
    const void* mats[] = {s.qkv_w, s.out_w, s.cross_q_w, s.cross_out_w, s.fc1_w, s.fc2_w,
                          s.self_k, s.self_v, s.cross_k, s.cross_v};
    for (const void* p : mats)
      if (reinterpret_cast<uintptr_t>(p) & 15u)
        return fw_fail(FW_EINVAL, "%s: layer %d: weights and caches must be 16-byte aligned", name, l);
    StepLayer& d = a.layer[l];
    auto h = [](const void* p) { return static_cast<const _Float16*>(p); };
    d.ln1_g = h(s.ln1_gamma); d.ln1_b = h(s.ln1_beta); d.qkv_w = h(s.qkv_w); d.qkv_b = h(s.qkv_b);
    d.out_w = h(s.out_w); d.out_b = h(s.out_b);
    d.ln2_g = h(s.ln2_gamma); d.ln2_b = h(s.ln2_beta); d.cq_w = h(s.cross_q_w); d.cq_b = h(s.cross_q_b);
    d.co_w = h(s.cross_out_w); d.co_b = h(s.cross_out_b);
    d.ln3_g = h(s.ln3_gamma); d.ln3_b = h(s.ln3_beta); d.fc1_w = h(s.fc1_w); d.fc1_b = h(s.fc1_b);
    d.fc2_w = h(s.fc2_w); d.fc2_b = h(s.fc2_b);
    d.eps1 = s.ln1_eps; d.eps2 = s.ln2_eps; d.eps3 = s.ln3_eps;
    d.self_k = static_cast<_Float16*>(s.self_k); d.self_v = static_cast<_Float16*>(s.self_v);
    d.cross_k = h(s.cross_k); d.cross_v = h(s.cross_v);
  }
  // the device-dependent checks last: every argument check above runs without a HIP call
  int grid = 0, dev = 0;
  if (const int st = step_sizes_check(name, n_layers, vocab, max_pos, enc_len, head != nullptr, prompt ? kPromptLen : 1,
                                      &grid))
    return st;
  if (hipGetDevice(&dev) != hipSuccess) return fw_fail(FW_EHIP, "%s: no device", name);
  if (head) {
    const fw_dec_head& hd = *head;
    a.has_head = 1;
    a.head = StepHead{static_cast<const _Float16*>(hd.ln_gamma), static_cast<const _Float16*>(hd.ln_beta), hd.ln_eps,
                      static_cast<const _Float16*>(hd.w), static_cast<const int8_t*>(hd.wq),
                      reinterpret_cast<const float2*>(hd.meta), hd.suppress, hd.tokens,
                      static_cast<_Float16*>(hd.y_out), hd.host_tokens, hd.n_eos, {}};
    for (int i = 0; i < hd.n_eos; ++i) a.head.eos[i] = hd.eos[i];
  }
  a.n_layers = n_layers;
  a.n_steps = n_steps;
  a.prompt = prompt;
  a.cur = cur;
  a.state = state;
  a.embed = static_cast<const _Float16*>(embed);
  a.pos_embed = static_cast<const _Float16*>(pos_embed);
  a.vocab = vocab;
  a.max_pos = max_pos;
  a.enc_len = enc_len;
  a.scale = scale;
  a.h_out = static_cast<_Float16*>(h_out);
  a.x_out = static_cast<_Float16*>(x_out);
  a.ws = static_cast<unsigned char*>(workspace);
  a.spin_limit = spin_limit;
  a.lm_res_rows = head && !prompt ? step_resident_rows(dev) : 0;
  if (prompt)
    hipLaunchKernelGGL(decoder_step_kernel<kPromptLen>, dim3(grid), dim3(kStepThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(decoder_step_kernel<1>, dim3(grid), dim3(kStepThreads), lm_res_bytes(a.lm_res_rows), stream, a);
  return fw_check_launch(name);
}

extern "C" int fw_decoder_step_layers(const fw_dec_layer* layers, int n_layers, const int64_t* cur,
                                      const int64_t* state, const void* embed, const void* pos_embed, int vocab,
                                      int max_pos, int enc_len, float scale, void* h_out, void* x_out,
                                      void* workspace, int64_t ws_bytes, int64_t spin_limit, hipStream_t stream) {
  return decoder_step_launch("decoder_step_layers", layers, n_layers, nullptr, nullptr, 1, const_cast<int64_t*>(cur),
                             const_cast<int64_t*>(state), embed, pos_embed, vocab, max_pos, enc_len, scale, h_out,
                             x_out, workspace, ws_bytes, spin_limit, stream);
}

extern "C" int fw_decoder_step(const fw_dec_layer* layers, int n_layers, const fw_dec_head* head, int n_steps,
                               int64_t* cur, int64_t* state, const void* embed, const void* pos_embed, int vocab,
                               int max_pos, int enc_len, float scale, void* workspace, int64_t ws_bytes,
                               int64_t spin_limit, hipStream_t stream) {
  if (!head) return fw_fail(FW_EINVAL, "decoder_step: null LM head");
  return decoder_step_launch("decoder_step", layers, n_layers, head, nullptr, n_steps, cur, state, embed, pos_embed,
                             vocab, max_pos, enc_len, scale, nullptr, nullptr, workspace, ws_bytes, spin_limit, stream);
}

extern "C" int fw_decoder_prompt(const fw_dec_layer* layers, int n_layers, const fw_dec_head* head,
                                 const int64_t* prompt, int n_prompt, int64_t* cur, int64_t* state, const void* embed,
                                 const void* pos_embed, int vocab, int max_pos, int enc_len, float scale,
                                 void* workspace, int64_t ws_bytes, int64_t spin_limit, hipStream_t stream) {
  if (!head || !prompt) return fw_fail(FW_EINVAL, "decoder_prompt: null LM head or prompt");
  if (n_prompt != kPromptLen) return fw_fail(FW_EINVAL, "decoder_prompt: n_prompt must be %d", kPromptLen);
  return decoder_step_launch("decoder_prompt", layers, n_layers, head, prompt, 1, cur, state, embed, pos_embed, vocab,
                             max_pos, enc_len, scale, nullptr, nullptr, workspace, ws_bytes, spin_limit, stream);
}
