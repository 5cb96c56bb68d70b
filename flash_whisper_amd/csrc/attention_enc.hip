// Whisper encoder self-attention for gfx950 (transformers models/whisper/modeling_whisper.py:284-358,
// SDPA path, fp16 in and out, fp32 softmax and accumulation), plus the transposed-V packing it reads.
// Built with MFMA results in VGPRs (-mllvm -amdgpu-mfma-vgpr-form): the softmax reads every score and
// the O accumulators are rescaled in place, which in the AGPR form costs a register move per value.
#include "lds_pipe.h"

namespace fw {
namespace {

// ------------------------------------------------------------------------------------------
// Encoder self-attention, flash style, non-causal, scale 1 (q is pre-scaled by the projection).
// Block = (head, 128 queries), 8 waves: 4 query groups of 32 x 2 key halves (even / odd 64-key tiles),
// so two waves share each SIMD and one's softmax overlaps the other's MFMAs; the halves' (m, l, O)
// are merged through LDS at the end. All waves share one LDS ring whose stages hold a tile pair. Per
// tile a wave computes S^T = K Q^T (keys x queries) with MFMA, so that every lane holds the scores
// of a single query column and the online-softmax max/sum need one cross-lane step (lane ^ 32).
// P^T is fed straight from the S^T accumulator layout as the B operand of O^T = V^T P^T.
//  - Inputs: q and k from the projection output qkv[seq, 3 * heads * 64]; V from a transposed copy
//    vt[heads][64][seq_pad] written by the projection's epilogue, whose key order inside every
//    16-key group has bits 2 and 3 of the key index swapped. With that order the 8 keys an MFMA
//    A-operand lane needs for V^T are one contiguous 16-byte chunk, and they are the keys the
//    same lane holds for P^T in the S^T accumulator (rows 8 (r / 4) + 4 g + (r % 4)).
//  - K tiles (64 keys x 128 B) and V^T tiles (64 d x 128 B) arrive by direct-to-LDS copies into a
//    ring of kEaStages stages, XOR-swizzled by 16-byte chunk like the GEMM tiles.
//  - Block ids are remapped so that the query blocks of a head run on one XCD and its K/V stay in
//    that XCD's L2.
// ------------------------------------------------------------------------------------------
constexpr int kEaQGroups = 4, kEaWaves = 2 * kEaQGroups, kEaQ = 32 * kEaQGroups, kEaKV = 64, kEaStages = 4;
constexpr int kEaTileBytes = kEaKV * 128;  // one K tile or one V^T tile

// The 4 waves of a key half fill one tile (K then V^T) of a ring stage; `wave` is 0..3 within the half.
__device__ __forceinline__ void ea_dma(const _Float16* kbase, int ld, const _Float16* vtbase, int seq_pad,
                                       int seq, int kv0, int wave, int lane, uint32_t stage) {
  const int rsub = lane >> 3, slot = lane & 7;
#pragma unroll
  for (int i = 0; i < 2; ++i) {  // K tile: wave fills 8-row blocks 2 wave and 2 wave + 1
    const int blk = 2 * wave + i, row = blk * 8 + rsub;
    const int key = min(kv0 + row, seq - 1);  // keys past seq are masked to -inf
    dma16(kbase + static_cast<size_t>(key) * ld + swz_slot(row, slot) * 8,
          __builtin_amdgcn_readfirstlane(stage + blk * 1024));
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {  // V^T tile: rows are head dims
    const int blk = 2 * wave + i, d = blk * 8 + rsub;
    dma16(vtbase + static_cast<size_t>(d) * seq_pad + kv0 + swz_slot(d, slot) * 8,
          __builtin_amdgcn_readfirstlane(stage + kEaTileBytes + blk * 1024));
  }
}

// The same copies for a tile whose 64 keys all lie below seq (every tile but a partial last one): the
// tile's first key only moves the scalar bases, and each lane keeps the byte offsets of its four chunks
// (rows of 64 keys or head dims times the row pitch, plus the swizzled chunk), so a stage costs no
// vector address arithmetic. The host keeps 64 rows of either operand within the 32-bit offsets.
struct EaCopyOffsets {
  uint32_t k[2], v[2];
};

__device__ __forceinline__ EaCopyOffsets ea_offsets(int ld, int seq_pad, int wave, int lane) {
  const int rsub = lane >> 3, slot = lane & 7;
  EaCopyOffsets o;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = (2 * wave + i) * 8 + rsub;  // key row of the K tile, head dim of the V^T tile
    o.k[i] = static_cast<uint32_t>((row * ld + swz_slot(row, slot) * 8) * 2);
    o.v[i] = static_cast<uint32_t>((row * seq_pad + swz_slot(row, slot) * 8) * 2);
  }
  return o;
}

__device__ __forceinline__ void ea_dma_full(const _Float16* kbase, int ld, const _Float16* vtbase, int kv0,
                                            const EaCopyOffsets& o, int wave, uint32_t stage) {
  const _Float16* kb = kbase + static_cast<size_t>(kv0) * ld;
  const _Float16* vb = vtbase + kv0;
#pragma unroll
  for (int i = 0; i < 2; ++i) dma16_s(o.k[i], kb, stage + (2 * wave + i) * 1024);
#pragma unroll
  for (int i = 0; i < 2; ++i) dma16_s(o.v[i], vb, stage + kEaTileBytes + (2 * wave + i) * 1024);
}

// Scores are kept in log2 units (x log2 e). The running max m used for p = exp2(s - m) is only moved
// when some lane of the wave sees a score more than kEaSlack above it, so p stays in [0, 2^kEaSlack]
// (exact in fp16's range) and the O/l rescale runs on few tiles instead of every tile.
constexpr float kEaSlack = 8.f;

struct EaState {
  f16v o[2];  // O^T blocks: d in [0, 32) and [32, 64)
  float m, l;
};

template <bool kMask>
__device__ __forceinline__ void ea_tile(const u32x4* kt, const u32x4* vtt, const h8v (&qf)[4], int kv0, int seq,
                                        int lr, int lg, EaState& st) {
  constexpr float kLog2e = 1.4426950408889634f;
  // S^T = K Q^T for two 32-key blocks.
  f16v s[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
#pragma unroll
    for (int r = 0; r < 16; ++r) s[b][r] = 0.f;
    const int row = 32 * b + lr;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const u32x4 u = kt[swz(row, 2 * k + lg)];
      s[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8v, u), qf[k], s[b], 0, 0, 0);
    }
  }
  float tmax = -INFINITY;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if constexpr (kMask) {
        if (kv0 + 32 * b + 8 * (r >> 2) + 4 * lg + (r & 3) >= seq) s[b][r] = -INFINITY;
      }
      tmax = fmaxf(tmax, s[b][r]);
    }
  tmax = xor_max<32>(tmax) * kLog2e;
  if (__builtin_amdgcn_ballot_w64(tmax > st.m + kEaSlack)) {  // wave-uniform
    const float m_new = fmaxf(st.m, tmax);
    const float corr = __builtin_amdgcn_exp2f(st.m - m_new);  // 0 on the first tile (m = -inf)
    st.l *= corr;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) st.o[b][r] *= corr;
    st.m = m_new;
  }
  h8v pf[2][2];  // P^T as B operand, [32-key block][k-step of 16 keys]
  float psum = 0.f;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      h2v ph;
      ph[0] = f2h(__builtin_amdgcn_exp2f(fmaf(s[b][r], kLog2e, -st.m)));
      ph[1] = f2h(__builtin_amdgcn_exp2f(fmaf(s[b][r + 1], kLog2e, -st.m)));
      psum = __builtin_amdgcn_fdot2(ph, h2v{static_cast<_Float16>(1.f), static_cast<_Float16>(1.f)}, psum, false);
      pf[b][r >> 3][r & 7] = ph[0];
      pf[b][r >> 3][(r & 7) + 1] = ph[1];
    }
  st.l += xor_add<32>(psum);
  // O^T[d][q] += sum_keys V^T[d][key] P^T[key][q]; k-step (b, hs) covers keys 32 b + 16 hs + [0, 16),
  // whose transposed-layout chunk for lane half lg is chunk 4 b + 2 hs + lg of the V^T row.
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int hs = 0; hs < 2; ++hs)
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const u32x4 u = vtt[swz(32 * db + lr, 4 * b + 2 * hs + lg)];
        st.o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8v, u), pf[b][hs], st.o[db], 0, 0, 0);
      }
}

__global__ void __launch_bounds__(kEaWaves * 64) encoder_attention_kernel(const _Float16* __restrict__ qkv,
                                                                         const _Float16* __restrict__ vt,
                                                                         _Float16* __restrict__ out, int seq,
                                                                         int heads) {
  constexpr int kPerStage = 4;                       // copies per thread per stage
  constexpr int kPairBytes = 2 * 2 * kEaTileBytes;   // K + V^T of two tiles
  __shared__ __align__(1024) u32x4 ring[kEaStages * kPairBytes / 16];
  static_assert(kEaStages * kPairBytes >= kEaQGroups * 64 * 34 * 4, "merge buffer fits in the ring");

  const int qblocks = (seq + kEaQ - 1) / kEaQ, nblk = qblocks * heads;
  const int bid = blockIdx.x, full = (nblk / 8) * 8;
  const int job = bid < full ? (bid % 8) * (full / 8) + bid / 8 : bid;
  const int head = job / qblocks, qb = job % qblocks;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wq = wave & (kEaQGroups - 1), half = wave / kEaQGroups;  // query group, key half (both wave-uniform)
  const int lr = lane & 31, lg = lane >> 5;
  const int ld = 3 * heads * kHeadDim, seq_pad = vt_pad(seq);
  const int q_row = qb * kEaQ + wq * 32 + lr;  // this lane's query column
  const _Float16* kbase = qkv + (heads + head) * kHeadDim;
  const _Float16* vtbase = vt + static_cast<size_t>(head) * kHeadDim * seq_pad;
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ring));

  // Q^T as B operand: lane holds Q[q_row][16 s + 8 lg .. + 7] for s = 0..3.
  h8v qf[4];
  {
    const _Float16* qp = qkv + static_cast<size_t>(min(q_row, seq - 1)) * ld + head * kHeadDim + 8 * lg;
#pragma unroll
    for (int k = 0; k < 4; ++k) qf[k] = *reinterpret_cast<const h8v*>(qp + 16 * k);
  }
  const int nt = seq_pad / kEaKV, npairs = (nt + 1) / 2;
  // Stage p holds tiles 2p (half 0) and 2p + 1 (half 1). A half whose tile is past the end copies the
  // last tile again, so every thread issues the same number of copies per stage (the vmcnt waits
  // count this thread's own copies).
  const EaCopyOffsets co = ea_offsets(ld, seq_pad, wq, lane);
  auto issue = [&](int p) {
    const int t = min(2 * p + half, nt - 1);
    const uint32_t stage = lds0 + (p % kEaStages) * kPairBytes + half * 2 * kEaTileBytes;
    if ((t + 1) * kEaKV <= seq)  // wave-uniform; both forms issue the same four copies
      ea_dma_full(kbase, ld, vtbase, t * kEaKV, co, wq, stage);
    else
      ea_dma(kbase, ld, vtbase, seq_pad, seq, t * kEaKV, wq, lane, stage);
  };
#pragma unroll
  for (int k = 0; k < kEaStages - 1; ++k)
    if (k < npairs) issue(k);

  EaState st;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) st.o[b][r] = 0.f;
  st.m = -INFINITY;
  st.l = 0.f;

  // Returns this half's K tile of pair p once every wave's copies of the pair have landed.
  auto next_pair = [&](int p) {
    wait_stages_ahead<kPerStage, kEaStages - 2>(min(kEaStages - 2, npairs - 1 - p));
    barrier_only();  // pair p visible to every wave; every wave is done with pair p - 1
    if (p + kEaStages - 1 < npairs) issue(p + kEaStages - 1);
    return ring + ((p % kEaStages) * kPairBytes + half * 2 * kEaTileBytes) / 16;
  };
  const int nfull = seq / kEaKV;  // tiles whose 64 keys are all valid; only the last tile may be partial
  for (int p = 0; p < npairs - 1; ++p) {  // both tiles of these pairs are full
    const u32x4* kt = next_pair(p);
    ea_tile<false>(kt, kt + kEaTileBytes / 16, qf, (2 * p + half) * kEaKV, seq, lr, lg, st);
  }
  {
    const u32x4* kt = next_pair(npairs - 1);
    const int t = 2 * (npairs - 1) + half;
    if (t < nfull)
      ea_tile<false>(kt, kt + kEaTileBytes / 16, qf, t * kEaKV, seq, lr, lg, st);
    else if (t < nt)
      ea_tile<true>(kt, kt + kEaTileBytes / 16, qf, t * kEaKV, seq, lr, lg, st);
  }

  // Merge the key halves: half 1 hands (m, l, O) through LDS to the wave of half 0 with the same
  // query group; lane for lane the registers describe the same query and head dims.
  lds_barrier();  // every wave is done with the ring
  float* mbuf = reinterpret_cast<float*>(ring) + (wq * 64 + lane) * 34;
  if (half == 1) {
    mbuf[0] = st.m;
    mbuf[1] = st.l;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) mbuf[2 + 16 * b + r] = st.o[b][r];
  }
  lds_barrier();
  if (half == 1 || q_row >= seq) return;
  const float m1 = mbuf[0], l1 = mbuf[1];
  const float m = fmaxf(st.m, m1);
  const float a0 = __builtin_amdgcn_exp2f(st.m - m), a1 = __builtin_amdgcn_exp2f(m1 - m);  // m1 may be -inf
  const float inv = 1.0f / (st.l * a0 + l1 * a1);
  _Float16* orow = out + static_cast<size_t>(q_row) * heads * kHeadDim + head * kHeadDim;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h4v v4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * j + e;
        v4[e] = f2h((st.o[db][r] * a0 + mbuf[2 + 16 * db + r] * a1) * inv);
      }
      *reinterpret_cast<h4v*>(orow + 32 * db + 8 * j + 4 * lg) = v4;
    }
}

// Transposed V for the attention kernel from a projection output (qkv v columns).
__global__ void __launch_bounds__(256) pack_vt_kernel(const _Float16* __restrict__ qkv, _Float16* __restrict__ vt,
                                                      int seq, int heads) {
  const int seq_pad = vt_pad(seq);
  const int i = blockIdx.x * 256 + threadIdx.x;  // over heads * 64 * seq_pad
  if (i >= heads * kHeadDim * seq_pad) return;
  const int pos = i % seq_pad, hd = i / seq_pad;  // hd = head * 64 + d
  const int t = vt_pos(pos);
  vt[i] = t < seq ? qkv[static_cast<size_t>(t) * 3 * heads * kHeadDim + 2 * heads * kHeadDim + hd]
                  : static_cast<_Float16>(0.f);
}


bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace
}  // namespace fw

using namespace fw;

extern "C" long long fw_encoder_vt_elems(int seq, int heads) {
  if (seq <= 0 || heads <= 0) return 0;
  return static_cast<long long>(heads) * kHeadDim * vt_pad(seq);
}

extern "C" int fw_encoder_pack_vt(const void* qkv, void* vt, int seq, int heads, hipStream_t stream) {
  if (!qkv || !vt) return fw_fail(FW_EINVAL, "encoder_pack_vt: null pointer");
  if (seq <= 0 || heads <= 0) return fw_fail(FW_EINVAL, "encoder_pack_vt: seq and heads must be positive");
  const long long n = fw_encoder_vt_elems(seq, heads);
  hipLaunchKernelGGL(pack_vt_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream,
                     static_cast<const _Float16*>(qkv), static_cast<_Float16*>(vt), seq, heads);
  return fw_check_launch("encoder_pack_vt");
}

extern "C" int fw_encoder_attention(const void* qkv, const void* vt, void* out, int seq, int heads,
                                    hipStream_t stream) {
  if (!qkv || !vt || !out) return fw_fail(FW_EINVAL, "encoder_attention: null pointer");
  if (seq <= 0 || heads <= 0) return fw_fail(FW_EINVAL, "encoder_attention: seq and heads must be positive");
  // 64 rows of K (pitch 3 heads 64) or of V^T (pitch vt_pad(seq)) within the copies' 32-bit byte offsets
  if (64LL * 3 * heads * kHeadDim * 2 >= (1LL << 32) || 64LL * vt_pad(seq) * 2 >= (1LL << 32))
    return fw_fail(FW_EINVAL, "encoder_attention: seq or heads too large");
  if (!aligned(qkv, 16) || !aligned(vt, 16) || !aligned(out, 8))
    return fw_fail(FW_EINVAL, "encoder_attention: qkv and vt must be 16-byte aligned, out 8-byte aligned");
  const int blocks = (seq + kEaQ - 1) / kEaQ * heads;
  hipLaunchKernelGGL(encoder_attention_kernel, dim3(blocks), dim3(kEaWaves * 64), 0, stream, static_cast<const _Float16*>(qkv),
                     static_cast<const _Float16*>(vt), static_cast<_Float16*>(out), seq, heads);
  return fw_check_launch("encoder_attention");
}
