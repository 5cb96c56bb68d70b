// Device code shared by the decoder kernels of decode.hip and the persistent decoder step of
// decode_step.hip: the residual + LayerNorm prologue, the GEMV row split, the split-K combine, the
// split attention's per-wave partials and the token finalize. Each .hip file that includes this header
// gets its own copy (internal linkage), so the kernels of both files run the same arithmetic.
#pragma once

#include "fw_common.h"

namespace fw {
namespace {

#ifndef FW_GEMV_WEIGHTS_NT
#define FW_GEMV_WEIGHTS_NT 0  // decoder weights may stay resident in the 256 MB MALL
#endif
#ifndef FW_LM_HEAD_NT
#define FW_LM_HEAD_NT 1
#endif
static_assert((FW_GEMV_WEIGHTS_NT == 0 || FW_GEMV_WEIGHTS_NT == 1) && (FW_LM_HEAD_NT == 0 || FW_LM_HEAD_NT == 1),
              "FW_GEMV_WEIGHTS_NT and FW_LM_HEAD_NT are switches (0 or 1)");
__device__ __forceinline__ uint4 ld_weights(const uint4* p) {
#if FW_GEMV_WEIGHTS_NT
  return ld_stream(p);
#else
  return *p;
#endif
}
__device__ __forceinline__ uint4 ld_lm_head(const uint4* p) {
#if FW_LM_HEAD_NT
  return ld_stream(p);
#else
  return *p;
#endif
}

// ------------------------------------------------------------------------------------------
// Residual + LayerNorm prologue shared by add_layernorm, the fused LN+GEMV and the LM head.
// Produces y = fp16(LN(r) * gamma + beta) for the 1280-wide hidden vector in `y_out` (LDS or
// global), where r = fp16(a + b) (b may be null) and a, b are either (h, x) or the embedding rows
// (embed[cur], pos_embed[pos]). Block 0 stores r to r_out when r_out is non-null.
// ------------------------------------------------------------------------------------------
// The inputs are loaded into registers by ln_load and consumed by ln_finish, so a kernel can issue
// its other global loads (the weight rows) in between: vector-memory counters retire in order, and
// inputs requested after the weights could not be used before the weights had arrived.
template <int NT>
struct LnRegs {
  static constexpr int kPairs = kHidden / 2;
  static constexpr int kPer = (kPairs + NT - 1) / NT;
  h2v a[kPer], b[kPer], g[kPer], be[kPer];
};

template <int NT>
__device__ __forceinline__ void ln_load(const _Float16* a, const _Float16* b, const _Float16* gamma,
                                        const _Float16* beta, LnRegs<NT>& in) {
  const h2v* a2 = reinterpret_cast<const h2v*>(a);
  const h2v* b2 = reinterpret_cast<const h2v*>(b);
  const h2v* g2 = reinterpret_cast<const h2v*>(gamma);
  const h2v* be2 = reinterpret_cast<const h2v*>(beta);
  const h2v zero = {static_cast<_Float16>(0.f), static_cast<_Float16>(0.f)};
#pragma unroll
  for (int i = 0; i < LnRegs<NT>::kPer; ++i) {
    const int idx = threadIdx.x + i * NT;
    const bool ok = idx < LnRegs<NT>::kPairs;
    in.a[i] = ok ? a2[idx] : zero;
    in.b[i] = (ok && b2) ? b2[idx] : zero;
    in.g[i] = ok ? g2[idx] : zero;
    in.be[i] = ok ? be2[idx] : zero;
  }
}

// kOwnSlots: the two reductions use red[0 .. NT/64) and red[NT/64 .. 2 NT/64) with one barrier each
// (the same sums); red must then hold 2 NT/64 floats and is free again after the caller's next barrier.
template <int NT, bool kOwnSlots = false>
__device__ __forceinline__ void ln_finish(const LnRegs<NT>& in, bool has_b, _Float16* r_out, float eps,
                                          _Float16* y_out, float* red) {
  constexpr int kPer = LnRegs<NT>::kPer;
  h2v* r2 = reinterpret_cast<h2v*>(r_out);
  h2v* y2 = reinterpret_cast<h2v*>(y_out);
  float2 r[kPer];
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int idx = threadIdx.x + i * NT;
    r[i] = make_float2(0.f, 0.f);
    if (idx < LnRegs<NT>::kPairs) {
      float rx = h2f(in.a[i].x), ry = h2f(in.a[i].y);
      if (has_b) {
        rx = round_h(rx + h2f(in.b[i].x));
        ry = round_h(ry + h2f(in.b[i].y));
      }
      r[i] = make_float2(rx, ry);
      sum += rx + ry;
      if (r2 && blockIdx.x == 0) {
        h2v o;
        o.x = f2h(rx);
        o.y = f2h(ry);
        r2[idx] = o;
      }
    }
  }
  const float mean = (kOwnSlots ? block_sum_once<NT>(sum, red) : block_sum<NT>(sum, red)) * (1.0f / kHidden);
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int idx = threadIdx.x + i * NT;
    if (idx < LnRegs<NT>::kPairs) {
      const float dx = r[i].x - mean, dy = r[i].y - mean;
      sq += dx * dx + dy * dy;
    }
  }
  const float var = (kOwnSlots ? block_sum_once<NT>(sq, red + NT / kWave) : block_sum<NT>(sq, red)) * (1.0f / kHidden);
  const float inv = rsqrtf(var + eps);
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int idx = threadIdx.x + i * NT;
    if (idx < LnRegs<NT>::kPairs) {
      h2v o;
      o.x = f2h((r[i].x - mean) * inv * h2f(in.g[i].x) + h2f(in.be[i].x));
      o.y = f2h((r[i].y - mean) * inv * h2f(in.g[i].y) + h2f(in.be[i].y));
      y2[idx] = o;
    }
  }
}

// ln_finish for NV vectors at once: the vectors' sums share each reduction round (two barriers in all
// instead of four per vector). Every value is reduced in the order block_sum uses (the wave butterfly,
// then the wave partials in wave order), so each vector's result is that of ln_finish on it alone.
// red holds 2 * NV * (NT / 64) floats.
template <int NT, int NV>
__device__ __forceinline__ void ln_finish_multi(const LnRegs<NT> (&in)[NV], bool has_b, _Float16* r_out, float eps,
                                                _Float16* y_out, float* red) {
  constexpr int kPer = LnRegs<NT>::kPer, kWaves = NT / kWave;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  float2 r[NV][kPer];
  float part[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    h2v* r2 = r_out ? reinterpret_cast<h2v*>(r_out + v * kHidden) : nullptr;
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int idx = threadIdx.x + i * NT;
      r[v][i] = make_float2(0.f, 0.f);
      if (idx < LnRegs<NT>::kPairs) {
        float rx = h2f(in[v].a[i].x), ry = h2f(in[v].a[i].y);
        if (has_b) {
          rx = round_h(rx + h2f(in[v].b[i].x));
          ry = round_h(ry + h2f(in[v].b[i].y));
        }
        r[v][i] = make_float2(rx, ry);
        sum += rx + ry;
        if (r2 && blockIdx.x == 0) {
          h2v o;
          o.x = f2h(rx);
          o.y = f2h(ry);
          r2[idx] = o;
        }
      }
    }
    part[v] = group_sum<kWave>(sum);
  }
  if (lane == 0) {
#pragma unroll
    for (int v = 0; v < NV; ++v) red[v * kWaves + wave] = part[v];
  }
  __syncthreads();
  float mean[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) s += red[v * kWaves + w];
    mean[v] = s * (1.0f / kHidden);
  }
  float* red2 = red + NV * kWaves;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int idx = threadIdx.x + i * NT;
      if (idx < LnRegs<NT>::kPairs) {
        const float dx = r[v][i].x - mean[v], dy = r[v][i].y - mean[v];
        sq += dx * dx + dy * dy;
      }
    }
    part[v] = group_sum<kWave>(sq);
  }
  if (lane == 0) {
#pragma unroll
    for (int v = 0; v < NV; ++v) red2[v * kWaves + wave] = part[v];
  }
  __syncthreads();
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) s += red2[v * kWaves + w];
    const float inv = rsqrtf(s * (1.0f / kHidden) + eps);
    h2v* y2 = reinterpret_cast<h2v*>(y_out + v * kHidden);
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int idx = threadIdx.x + i * NT;
      if (idx < LnRegs<NT>::kPairs) {
        h2v o;
        o.x = f2h((r[v][i].x - mean[v]) * inv * h2f(in[v].g[i].x) + h2f(in[v].be[i].x));
        o.y = f2h((r[v][i].y - mean[v]) * inv * h2f(in[v].g[i].y) + h2f(in[v].be[i].y));
        y2[idx] = o;
      }
    }
  }
}

template <int NT>
__device__ __forceinline__ void ln_prologue(const _Float16* a, const _Float16* b, _Float16* r_out,
                                            const _Float16* gamma, const _Float16* beta, float eps,
                                            _Float16* y_out, float* red) {
  LnRegs<NT> in;
  ln_load<NT>(a, b, gamma, beta, in);
  ln_finish<NT>(in, b != nullptr, r_out, eps, y_out, red);
}

// Token and position embedding rows of vector v of a batch: token cur[v] at position state[0] + v.
// The token and position embedding rows of token tok at position pos (both clamped into range).
__device__ __forceinline__ void embed_rows_of(int64_t tok, int64_t pos, const _Float16* embed, const _Float16* pos_embed,
                                              int vocab, int max_pos, const _Float16** a, const _Float16** b) {
  tok = tok < 0 ? 0 : (tok >= vocab ? vocab - 1 : tok);
  pos = pos < 0 ? 0 : (pos >= max_pos ? max_pos - 1 : pos);
  *a = embed + tok * kHidden;
  *b = pos_embed + pos * kHidden;
}

__device__ __forceinline__ void embed_rows(const int64_t* cur, const int64_t* state, const _Float16* embed,
                                           const _Float16* pos_embed, int vocab, int max_pos, const _Float16** a,
                                           const _Float16** b, int v = 0) {
  embed_rows_of(cur[v], state[0] + v, embed, pos_embed, vocab, max_pos, a, b);
}

template <int K>
struct RowSplit {
  static constexpr int kChunksRow = K / 8;
  static constexpr int kLPR = (K == kHidden) ? 32 : 64;
  static constexpr int kC = kChunksRow / kLPR;
  static constexpr int kRPW = kWave / kLPR;
  static_assert(kChunksRow % kLPR == 0, "row must split evenly over the lanes");
};

struct LnArgs {
  const _Float16* h;
  const _Float16* x;
  _Float16* h_out;
  const _Float16* gamma;
  const _Float16* beta;
  float eps;
  const int64_t* cur;
  const int64_t* state;
  const _Float16* embed;
  const _Float16* pos_embed;
  int vocab;
  int max_pos;
};

// Split-K attention partials consumed by the GEMV that follows the attention (the out projection):
// the combine of the reference's decode_attention_combine_kernel (whisper_kernels.cu:191-213) runs
// as that GEMV's prologue, so the attention output never makes a round trip through a separate
// launch. `len_state` (self attention) limits the combine to the splits that held keys.
struct CombineArgs {
  const float* part_m;
  const float* part_l;
  const float* part_acc;
  const int64_t* len_state;
  int max_len;
  int split_keys;
  int nsplit;
  int heads;
  int pos_offset;  // vector v of a batch attends at position len_state[0] + v

  // The partials of vector v of a batch (laid out vector-major, heads * nsplit slots each).
  __device__ CombineArgs vec(int v) const {
    CombineArgs c = *this;
    const size_t slots = static_cast<size_t>(heads) * nsplit;
    c.part_m += v * slots;
    c.part_l += v * slots;
    c.part_acc += v * slots * kHeadDim;
    c.pos_offset = v;
    return c;
  }
};

constexpr int kMaxCombineSplits = 8;   // splits per head the combine prologue merges
constexpr int kMaxCombineHeads = 32;

__device__ __forceinline__ int active_splits(const int64_t* len_state, int max_len, int split_keys, int nsplit,
                                             int pos_offset = 0) {
  if (!len_state) return nsplit;
  int64_t p = len_state[0] + pos_offset;
  p = p < 0 ? 0 : (p >= max_len ? max_len - 1 : p);
  return static_cast<int>((p + split_keys) / split_keys);  // ceil((p + 1) / split_keys)
}

// x[h * 64 + d] = fp16(sum_s acc[h, s, d] e^(m_s - M) / sum_s l_s e^(m_s - M)), splits with l = 0 skipped
// (the arithmetic of the combine launch). combine_load requests every partial a thread needs;
// combine_finish merges them once they have landed.
template <int NT>
struct CombineRegs {
  static constexpr int kPer = (kHidden + NT - 1) / NT;
  float pm[kMaxCombineSplits], pl[kMaxCombineSplits];
  float pa[kPer][kMaxCombineSplits];
  int active;
};

template <int NT>
__device__ __forceinline__ void combine_load(const CombineArgs& c, CombineRegs<NT>& r) {
  constexpr int S = kMaxCombineSplits;
  r.active = active_splits(c.len_state, c.max_len, c.split_keys, c.nsplit, c.pos_offset);
  const int h0 = threadIdx.x;  // threads below `heads` also own one head's weights
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const bool ok = h0 < c.heads && s < r.active;
    r.pm[s] = ok ? c.part_m[h0 * c.nsplit + s] : -INFINITY;
    r.pl[s] = ok ? c.part_l[h0 * c.nsplit + s] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < CombineRegs<NT>::kPer; ++i) {
    const int j = threadIdx.x + i * NT;
    const int h = j / kHeadDim, d = j % kHeadDim;
#pragma unroll
    for (int s = 0; s < S; ++s)
      r.pa[i][s] = (j < c.heads * kHeadDim && s < r.active)
                       ? c.part_acc[(static_cast<size_t>(h) * c.nsplit + s) * kHeadDim + d] : 0.f;
  }
}

template <int NT>
__device__ __forceinline__ void combine_finish(const CombineArgs& c, const CombineRegs<NT>& r, _Float16* x,
                                               float* wgt, float* den_lds) {
  constexpr int S = kMaxCombineSplits;
  static_assert(NT >= kMaxCombineHeads, "one thread per head computes the split weights");
  if (threadIdx.x < c.heads) {
    const int h = threadIdx.x;
    float m = -INFINITY;
#pragma unroll
    for (int s = 0; s < S; ++s) m = fmaxf(m, r.pm[s]);
    float den = 0.f;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const float w = r.pl[s] > 0.f ? __expf(r.pm[s] - m) : 0.f;
      wgt[h * S + s] = w;
      den = fmaf(r.pl[s], w, den);
    }
    den_lds[h] = den;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < CombineRegs<NT>::kPer; ++i) {
    const int j = threadIdx.x + i * NT;
    if (j < c.heads * kHeadDim) {
      const int h = j / kHeadDim;
      float num = 0.f;
#pragma unroll
      for (int s = 0; s < S; ++s)
        if (wgt[h * S + s] != 0.f) num = fmaf(r.pa[i][s], wgt[h * S + s], num);
      x[j] = f2h(num / den_lds[h]);
    }
  }
}

constexpr int kModePlain = 0, kModeLn = 1, kModeCombine = 2;

// Stands in for a missing bias: a load from it replaces a branch around the bias load (a branch
// whose join would wait for every load issued before it).
__device__ _Float16 g_zero_half = static_cast<_Float16>(0.f);

struct FinArgs {
  int64_t* tokens;
  int64_t* state;
  int64_t* cur;
  int max_pos;
};

// The finalize with the packed maximum b and the state words already read: n = state[1] (tokens so
// far), p = state[0] (position). Returns the token and the new state words it wrote.
struct FinOut {
  int64_t tok, n, pos;
};
__device__ __forceinline__ FinOut finalize_known(unsigned long long b, int64_t n, int64_t p, const FinArgs& f) {
  FinOut o;
  o.tok = static_cast<int64_t>(0xFFFFFFFFu - static_cast<unsigned int>(b & 0xFFFFFFFFull));
  if (n < f.max_pos) f.tokens[n] = o.tok;
  o.n = n < f.max_pos ? n + 1 : n;
  o.pos = p + 1 < f.max_pos ? p + 1 : f.max_pos - 1;
  f.state[1] = o.n;
  f.state[0] = o.pos;
  *f.cur = o.tok;
  return o;
}

__device__ __forceinline__ void finalize_token(unsigned long long* best, const FinArgs& f) {
  const unsigned long long b = *best;
  *best = 0ull;
  finalize_known(b, f.state[1], f.state[0], f);
}

// ------------------------------------------------------------------------------------------
// Split-K single-query attention (flash-decoding; reference decode_attention_split_kernel,
// whisper_kernels.cu:102-189). Block (split, head) covers split_keys keys. A key row is 64 fp16 =
// 8 lanes x 16 bytes, so one wave scores 8 keys per pass and a 256-thread block 32 keys. Scores,
// max and exp-sum stay in fp32; the block writes its (m, l, acc[64]) partial and a second launch
// merges them (reference decode_attention_combine_kernel, :191-213). Self mode reads
// len = state[0] + 1 from device memory and the block owning row pos writes k_new/v_new into the
// cache while using the new row directly.
// ------------------------------------------------------------------------------------------
struct AttnArgs {
  const _Float16* q;
  _Float16* k;
  _Float16* v;
  const _Float16* k_new;
  const _Float16* v_new;
  const int64_t* len_state;
  int max_len;
  int split_keys;
  float scale;
  float* part_m;
  float* part_l;
  float* part_acc;
  _Float16* out;
  // batches of queries (split kernel, grid.z): query z is q + z * q_stride at position len_state[0] + z,
  // and its fresh K/V row is k_new / v_new + z * kv_stride
  int q_stride;
  int kv_stride;
};

__device__ __forceinline__ int attn_pos(const AttnArgs& a) {
  if (!a.len_state) return -1;
  const int64_t p = a.len_state[0];
  return static_cast<int>(p < 0 ? 0 : (p >= a.max_len ? a.max_len - 1 : p));
}

// Splits of up to 256 keys (the cross attention): FW_ATTN256_P passes of 8 keys per wave, 32 / P waves.
// 4 waves of 64 keys measured 0.9 us faster per decoder step than 8 waves of 32 on MI355X (34 launches).
#ifndef FW_ATTN256_P
#define FW_ATTN256_P 8
#endif
static_assert(FW_ATTN256_P >= 4 && 32 % FW_ATTN256_P == 0,
              "FW_ATTN256_P: whole waves of P passes over 256 keys, at most 8 waves");

// The scores, softmax and P.V of one wave's keys of a split (MAXP passes of 8 keys, keys at or past w1
// masked): the wave's (max, exp-sum, value sum) go to wm, wl and wacc_row for split_merge_store. Lane
// l holds key w0 + 8 p + l / 8 of pass p and chunk l % 8 of its row; fp32 throughout, the scale
// applied after the dot. A masked key's K and V registers may hold any row (callers load a clamped
// row rather than branch around the load, which would wait for every earlier load at the join): its
// score is -inf and its V is taken as zero, so it adds exactly what a zero row adds.
template <int MAXP>
__device__ __forceinline__ void split_wave_partial(const uint4 (&kr)[MAXP], const uint4 (&vr)[MAXP], const uint4& qc,
                                                   int w0, int w1, float scale, float* wm, float* wl,
                                                   float* wacc_row) {
  const int lane = threadIdx.x & 63, ks = lane >> 3, c = lane & 7;
  float sc[MAXP];
  float mx = -INFINITY;
#pragma unroll
  for (int p = 0; p < MAXP; ++p) {
    sc[p] = group_sum<8>(dot8(kr[p], qc, 0.f)) * scale;
    if (w0 + p * 8 + ks >= w1) sc[p] = -INFINITY;
    mx = fmaxf(mx, sc[p]);
  }
  mx = group_max<64>(mx);
  float acc[8], psum = 0.f;
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = 0.f;
  if (mx != -INFINITY) {
    if (w0 + MAXP * 8 <= w1) {  // wave-uniform: every key is live, so no V needs masking (the same sums)
#pragma unroll
      for (int p = 0; p < MAXP; ++p) {
        const float pj = __expf(sc[p] - mx);
        psum += pj;
        const h2v* v2 = reinterpret_cast<const h2v*>(&vr[p]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {  // fma with the fp16 operand widened in the instruction (v_fma_mix_f32)
          acc[2 * t] = fmaf(pj, h2f(v2[t].x), acc[2 * t]);
          acc[2 * t + 1] = fmaf(pj, h2f(v2[t].y), acc[2 * t + 1]);
        }
      }
    } else {
#pragma unroll
      for (int p = 0; p < MAXP; ++p) {
        const float pj = __expf(sc[p] - mx);
        psum += pj;
        const h2v* v2 = reinterpret_cast<const h2v*>(&vr[p]);
        const bool live = w0 + p * 8 + ks < w1;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          acc[2 * t] = fmaf(pj, live ? h2f(v2[t].x) : 0.f, acc[2 * t]);
          acc[2 * t + 1] = fmaf(pj, live ? h2f(v2[t].y) : 0.f, acc[2 * t + 1]);
        }
      }
    }
  }
  psum = xor_add<32>(xor_add<16>(xor_add<8>(psum)));
  const float o = sum8_transposed(acc);  // element c * 8 + sum8_index(lane), summed over the 8 key slots
  if (lane == 0) {
    *wm = mx;
    *wl = psum;
  }
  wacc_row[c * 8 + sum8_index(lane)] = o;
}

// The split's (m, l, acc[d]) from the NW wave partials, merged in wave order (after a block barrier).
template <int NW>
__device__ __forceinline__ void split_merge(const float* wm, const float* wl, const float (*wacc)[kHeadDim], int d,
                                            float& m, float& l, float& o) {
  // every wave's values first (one batch of LDS reads), then the merge with selects: a branch per wave
  // made each read a round trip of its own
  float pm[NW], pl[NW], pa[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    pm[w] = wm[w];
    pl[w] = wl[w];
    pa[w] = wacc[w][d];
  }
  m = -INFINITY;
#pragma unroll
  for (int w = 0; w < NW; ++w) m = fmaxf(m, pm[w]);
  l = 0.f;
  o = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const float wgt = __expf(pm[w] - m);
    const bool live = pl[w] > 0.f;
    l = live ? fmaf(pl[w], wgt, l) : l;
    o = live ? fmaf(pa[w], wgt, o) : o;
  }
}

// After a block barrier: thread d < 64 merges the NW wave partials in wave order and stores the
// split's (m, l, acc[d]) at `slot`.
template <int NW>
__device__ __forceinline__ void split_merge_store(const float* wm, const float* wl, const float (*wacc)[kHeadDim],
                                                  const AttnArgs& a, int slot) {
  const int tid = threadIdx.x;
  if (tid < kHeadDim) {
    float m, l, o;
    split_merge<NW>(wm, wl, wacc, tid, m, l, o);
    a.part_acc[static_cast<size_t>(slot) * kHeadDim + tid] = o;
    if (tid == 0) {
      a.part_m[slot] = m;
      a.part_l[slot] = l;
    }
  }
}

// ------------------------------------------------------------------------------------------
// The int8 pre-pass of the LM head (the soundness argument is at lm_head_q8_kernel in decode.hip).
// ------------------------------------------------------------------------------------------
constexpr int kQ8Chunks = kHidden / 16;           // 16-byte int8 chunks per row (80)
constexpr int kQ8Lpr = 16;                        // lanes per row in the int8 pass
constexpr int kQ8C = kQ8Chunks / kQ8Lpr;          // chunks per lane (5)
constexpr int kQ8YMax = 127 * 128;                // |y_int| bound: digits hi in [-127, 127], lo in [-64, 63]
constexpr float kQ8Gamma = 7.7e-5f;               // >= 1280 * 2^-24 / (1 - 1280 * 2^-24)

__device__ __forceinline__ int xor_add_i16(int v) {
  // integer butterfly over 16 lanes (partners 8, 4, 2, 1), exact
  v += __builtin_bit_cast(int, xor_lane<8>(__builtin_bit_cast(float, v)));
  v += __builtin_bit_cast(int, xor_lane<4>(__builtin_bit_cast(float, v)));
  v += __builtin_bit_cast(int, xor_lane<2>(__builtin_bit_cast(float, v)));
  v += __builtin_bit_cast(int, xor_lane<1>(__builtin_bit_cast(float, v)));
  return v;
}

__device__ __forceinline__ int dot16_i8(const uint4& a, const uint4& b, int acc) {
  acc = __builtin_amdgcn_sdot4(static_cast<int>(a.x), static_cast<int>(b.x), acc, false);
  acc = __builtin_amdgcn_sdot4(static_cast<int>(a.y), static_cast<int>(b.y), acc, false);
  acc = __builtin_amdgcn_sdot4(static_cast<int>(a.z), static_cast<int>(b.z), acc, false);
  acc = __builtin_amdgcn_sdot4(static_cast<int>(a.w), static_cast<int>(b.w), acc, false);
  return acc;
}

// The bound of the int8 pre-pass in fp32. With y's scale t, ||y|| <= ny and ||eta|| <= neta (eta = y - t
// y_int), a row with scale s, error bound e and exact digit dots ah, al (y_int = 128 hi + lo) has its fp32
// logit X within r = ny e + (neta + gamma ny)(127 s sqrt(1280) + e) of A = s t (128 ah + al). Written
// r = e a_e + s b_s with a_e = ny + k, b_s = k 127 sqrt(1280), k = neta + gamma ny (per step). In fp32:
// n = 128 ah + al is within 2^-24 (128 |ah| + |n|) (ah rounded once, al exact, one fma), so s t n within
// 3 2^-24 |s t| (128 |ah| + |n|); that term is covered 8 times over, r's six roundings of positive terms by
// the factor 1 + 2^-18, and the last add's rounding by what is left of both. So ub >= A + r and
// lb <= A - r: the interval holds the interval of the exact bound, and every argument made for that one
// (the candidate rule) holds for it.
struct Q8Step {
  float t, a_e, b_s;
};
__device__ __forceinline__ Q8Step q8_step(float amax, float ysq) {
  // |y|: an fp32 sum of <= 1280 non-negative terms is within 1280 * 2^-24 < 2^-10 relative. |eta|: with
  // t and 1 / t each rounded once and y / t = y * tinv to within 3 * 2^-24 of |y / t| <= kQ8YMax
  // (< 0.003), every |y_i - t y_int_i| <= 0.503 t (one more rounding included).
  const float t = amax > 0.f ? amax / static_cast<float>(kQ8YMax) : 1.0f;
  const float ny = sqrtf(ysq) * (1.0f + 0x1p-9f);
  const float neta = amax > 0.f ? 0.51f * t * 35.77708764f : 0.f;  // sqrt(1280)
  const float k = fmaf(kQ8Gamma, ny, neta);
  return {t, ny + k, k * 4543.6901f};                               // 127 sqrt(1280)
}
__device__ __forceinline__ void q8_bounds(int ah, int al, float2 m, const Q8Step& q, float& ub, float& lb) {
  const float st = m.x * q.t;
  const float fh = static_cast<float>(ah);
  const float n = fmaf(128.0f, fh, static_cast<float>(al));
  const float av = st * n;
  const float err = (st * 0x1p-21f) * fmaf(128.0f, fabsf(fh), fabsf(n));
  const float r = fmaf(fmaf(m.y, q.a_e, m.x * q.b_s), 1.0f + 0x1p-18f, err + 1e-30f);
  ub = av + r;
  lb = av - r;
}

// Smallest X that can still tie or beat a row whose fp32 logit is at least T once both are rounded to
// fp16 (round to nearest even; logits at or beyond 65520 round to +-inf and tie there).
__device__ __forceinline__ float q8_threshold(float t) {
  if (!(t > -65504.0f)) return -INFINITY;  // also NaN: keep every row
  return fminf(t - (fabsf(t) * 0x1p-9f + 0x1p-23f), 65504.0f);
}

}  // namespace
}  // namespace fw
