/*
 * flash_whisper_amd C ABI: batch-1 Whisper-large-v3-turbo hot path on MI355X (gfx950).
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t, enqueues its
 * kernels on that stream without synchronising or allocating, and returns a status:
 *   FW_OK (0)       success (launch enqueued),
 *   FW_EINVAL (-1)  argument validation failed before any launch,
 *   FW_EHIP (-2)    the HIP runtime reported an error for a launch.
 * fw_last_error() returns the calling thread's last error message.
 *
 * fp16 tensors are IEEE binary16 ("half"), passed as void*. All tensors are dense and
 * row-major (C-contiguous). Reference citations are to sp4s-s/flash_whisper.
 */
#ifndef FLASH_WHISPER_H_
#define FLASH_WHISPER_H_

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FW_OK 0
#define FW_EINVAL (-1)
#define FW_EHIP (-2)

/* GEMV epilogue activations. */
#define FW_ACT_NONE 0
#define FW_ACT_GELU 1

/* Encoder GEMM epilogues (applied to fp32 acc, rounding points as in HF fp16 Whisper). */
#define FW_EPI_BIAS 0          /* out = fp16(acc + b)                                   */
#define FW_EPI_BIAS_GELU 1     /* out = fp16(gelu(fp16(acc + b)))                       */
#define FW_EPI_BIAS_RESID 2    /* out = fp16(res + fp16(acc + b))   (out may alias res) */
#define FW_EPI_BIAS_RESID_CLAMP 3 /* as RESID, then clamp to +-(65504 - 1000): +-64512 in fp16 */
#define FW_EPI_BIAS_GELU_POS 4 /* out = fp16(fp16(gelu(fp16(acc + b))) + res)           */
#define FW_EPI_SCALE_Q 5       /* columns < q_cols: fp16(fp16(acc + b) * 0.125); k/v as BIAS */

const char* fw_last_error(void);
int fw_version(void);

/* ---- reference ops (custom/kernels/whisper_kernels.cu) ---------------------------------- */

/* Replaces lm_head_argmax (whisper_kernels.cu:278-289, kernel :28-86).
 * best <- max(best, pack(fp16(y . w[v]), v)) over v with !suppress[v]; ties -> lower index.
 * y fp16[hidden], w fp16[vocab, hidden], suppress u8/bool[vocab], best u64[1]. hidden == 1280. */
int fw_lm_head_argmax(const void* y, const void* w, const uint8_t* suppress, int vocab, int hidden,
                      uint64_t* best, hipStream_t stream);

/* Replaces argmax_finalize (whisper_kernels.cu:291-298, kernel :88-100).
 * tok <- unpack(best); best <- 0; if state[1] < max_pos: tokens[state[1]] <- tok;
 * state[1] <- min(state[1] + 1, max_pos); state[0] <- min(state[0] + 1, max_pos - 1); cur <- tok. */
int fw_argmax_finalize(uint64_t* best, int64_t* tokens, int64_t* state, int64_t* cur, int max_pos,
                       hipStream_t stream);

/* Replaces decode_attention (whisper_kernels.cu:300-339, kernels :102-213): split-K single-query
 * attention, 64 keys per split, then a combine launch. q fp16[heads*64]; k, v fp16[heads, max_len, 64];
 * out fp16[heads*64]. Self mode: len_state, k_new, v_new all non-NULL, len = len_state[0] + 1, and the
 * row len_state[0] of k/v is overwritten with k_new/v_new (fp16[heads*64]). Cross mode: all three
 * NULL, len = max_len. part_m/part_l fp32[ws_slots], part_acc fp32[ws_slots*64],
 * ws_slots >= heads * ceil(max_len / 64). */
int fw_decode_attention(const void* q, void* k, void* v, void* out, const int64_t* len_state,
                        const void* k_new, const void* v_new, int heads, int max_len, float* part_m,
                        float* part_l, float* part_acc, int64_t ws_slots, float scale, hipStream_t stream);

/* fw_decode_attention without the workspace arguments, for callers that cannot allocate (code under
 * hipGraph capture, tight serving loops, harnesses that forbid hipMalloc); it has no counterpart in
 * the reference. Same kernels and the same result, bit for bit. The split partials live in a static
 * device array of this library: FW_NOALLOC_ATTN_SLOTS (head, split) slots, 528 KiB on each GPU the
 * library runs on, held until the process ends. heads * ceil(max_len / 64) above FW_NOALLOC_ATTN_SLOTS
 * fails with FW_EINVAL before any launch. The array's address on a device is looked up at the first
 * call on that device; no call allocates or frees memory. Calls on one GPU share the array: calls that
 * overlap on one GPU (different streams) race. */
#define FW_NOALLOC_ATTN_SLOTS 2048
int fw_decode_attention_noalloc(const void* q, void* k, void* v, void* out, const int64_t* len_state,
                                const void* k_new, const void* v_new, int heads, int max_len, float scale,
                                hipStream_t stream);

/* Replaces add_layernorm (whisper_kernels.cu:341-356, kernel :215-267).
 * If x != NULL: h <- fp16(h + x). Then y <- fp16(LN(h) * gamma + beta), two-pass fp32 statistics.
 * h, x, gamma, beta, y fp16[n]; n == 1280. */
int fw_add_layernorm(void* h, const void* x, const void* gamma, const void* beta, void* y, int n,
                     float eps, hipStream_t stream);

/* ---- fused decoder ops (no reference counterpart; they fuse the reference's step,
 *      custom/model.py:107-123, into fewer launches) ------------------------------------- */

/* Token + position embedding (custom/model.py:110): h <- fp16(embed[cur[0]] + pos_embed[state[0]]).
 * Indices are clamped into [0, vocab) and [0, max_pos). */
int fw_embed(const int64_t* cur, const int64_t* state, const void* embed, const void* pos_embed, int vocab,
             int max_pos, void* h, int hidden, hipStream_t stream);

/* out[n] <- act(fp16(w[n, :] . x + bias[n])) for n < n_out; w fp16[n_out, k_in], k_in in {1280, 5120}.
 * Replaces F.linear (+F.gelu) at custom/model.py:114,116,117,119,120. bias may be NULL. */
int fw_gemv(const void* x, const void* w, const void* bias, void* out, int n_out, int k_in, int act,
            hipStream_t stream);

/* Fused residual + LayerNorm + GEMV (custom/model.py:113-120 chains add_layernorm into F.linear).
 * r <- fp16(h + x) (x may be NULL: r <- h); if h_out != NULL, h_out <- r (h_out must not alias h);
 * y <- fp16(LN(r) * gamma + beta); out <- act(fp16(w . y + bias)). k_in == 1280.
 * Embedding mode: if cur != NULL, r <- fp16(embed[cur[0]] + pos_embed[state[0]]) instead (h, x ignored). */
int fw_ln_gemv(const void* h, const void* x, void* h_out, const void* gamma, const void* beta, float eps,
               const int64_t* cur, const int64_t* state, const void* embed, const void* pos_embed, int vocab,
               int max_pos, const void* w, const void* bias, void* out, int n_out, int k_in, int act,
               hipStream_t stream);

/* The LM head's final LayerNorm alone: y <- fp16(LN(fp16(h + x)) * gamma + beta) (x may be NULL) with
 * the reduction order of the 1024-thread LM-head kernels (fw_lm_head_argmax_fused, fw_lm_head_argmax_q8),
 * so y is the vector those kernels score, bit for bit. Replaces the final add_layernorm of
 * custom/model.py:121 at that order. n == 1280. */
int fw_final_layernorm(const void* h, const void* x, const void* gamma, const void* beta, void* y, int n, float eps,
                       hipStream_t stream);

/* Decode attention in one launch (same contract as fw_decode_attention, no workspace): one
 * 1024-thread block per head covers all keys and merges its 16 wave partials on chip. */
int fw_decode_attention_fused(const void* q, void* k, void* v, void* out, const int64_t* len_state,
                              const void* k_new, const void* v_new, int heads, int max_len, float scale,
                              hipStream_t stream);

/* The split half of fw_decode_attention alone: per (head, split) flash-decoding partials
 * (m, l, acc[64]) of split_keys keys each (multiple of 8, <= 256) into part_m/part_l/part_acc;
 * self mode writes the k_new/v_new cache row as fw_decode_attention does. */
int fw_attention_split(const void* q, void* k, void* v, const int64_t* len_state, const void* k_new,
                       const void* v_new, int heads, int max_len, int split_keys, float* part_m, float* part_l,
                       float* part_acc, int64_t ws_slots, float scale, hipStream_t stream);

/* Attention combine + output projection in one launch: x = combine(partials of fw_attention_split
 * with the same heads/max_len/split_keys; len_state limits self attention to the filled splits),
 * rounded to fp16 exactly as the fw_decode_attention output, then out <- fp16(w . x + bias).
 * heads * 64 == 1280, heads <= 32, ceil(max_len / split_keys) <= 8. */
int fw_attn_out_gemv(const float* part_m, const float* part_l, const float* part_acc, int64_t ws_slots,
                     const int64_t* len_state, int heads, int max_len, int split_keys, const void* w,
                     const void* bias, void* out, int n_out, hipStream_t stream);

/* ---- batched prompt (no reference counterpart: custom/model.py:196-207 runs the prompt one
 *      token per step; these run its nv <= 4 positions through each layer in one launch per op) --- */

/* fw_gemv on nv input vectors: x holds nv rows of k_in, out nv rows of n_out. Each row's result is
 * bit-identical to fw_gemv on that row. */
int fw_gemv_batch(const void* x, const void* w, const void* bias, void* out, int n_out, int k_in, int act, int nv,
                  hipStream_t stream);

/* fw_ln_gemv on nv vectors: h, x, h_out hold nv rows of 1280, out nv rows of n_out. Embedding mode
 * takes token cur[v] at position state[0] + v for vector v. Each vector's results are bit-identical
 * to fw_ln_gemv on it. */
int fw_ln_gemv_batch(const void* h, const void* x, void* h_out, const void* gamma, const void* beta, float eps,
                     const int64_t* cur, const int64_t* state, const void* embed, const void* pos_embed, int vocab,
                     int max_pos, const void* w, const void* bias, void* out, int n_out, int k_in, int act, int nv,
                     hipStream_t stream);

/* fw_attention_split for nq queries: query z is q + z * q_stride (elements) and, in self mode, sits at
 * position len_state[0] + z with its fresh K/V row at k_new / v_new + z * kv_stride; it attends to the
 * cached rows before len_state[0] and to the fresh rows of queries 0..z, and its row is written to the
 * cache. Partials are laid out query-major (nq * heads * splits slots), ready for
 * fw_attn_out_gemv_batch. Strides are multiples of 8 and at least heads * 64; nq <= 4. */
int fw_attention_split_batch(const void* q, void* k, void* v, const int64_t* len_state, const void* k_new,
                             const void* v_new, int heads, int max_len, int split_keys, float* part_m, float* part_l,
                             float* part_acc, int64_t ws_slots, float scale, int nq, int q_stride, int kv_stride,
                             hipStream_t stream);

/* fw_attn_out_gemv on the partials of nv queries from fw_attention_split_batch: vector v combines
 * the splits of position len_state[0] + v (self mode); out holds nv rows of n_out. */
int fw_attn_out_gemv_batch(const float* part_m, const float* part_l, const float* part_acc, int64_t ws_slots,
                           const int64_t* len_state, int heads, int max_len, int split_keys, const void* w,
                           const void* bias, void* out, int n_out, int nv, hipStream_t stream);

/* One decoder layer's tensors for fw_decoder_step_layers (fp16; weights in torch Linear layout).
 * qkv_w [3 * 1280, 1280] packed [q; k; v] with bias [b_q; 0; b_v] (custom/model.py:81-91); out_w,
 * cross_q_w, cross_out_w [1280, 1280]; fc1_w [5120, 1280]; fc2_w [1280, 5120]; null biases read as 0.
 * self_k / self_v [20, max_pos, 64] (this layer's KV cache), cross_k / cross_v [20, enc_len, 64]. */
typedef struct fw_dec_layer {
  const void *ln1_gamma, *ln1_beta, *qkv_w, *qkv_b, *out_w, *out_b;
  const void *ln2_gamma, *ln2_beta, *cross_q_w, *cross_q_b, *cross_out_w, *cross_out_b;
  const void *ln3_gamma, *ln3_beta, *fc1_w, *fc1_b, *fc2_w, *fc2_b;
  float ln1_eps, ln2_eps, ln3_eps;
  void *self_k, *self_v;
  const void *cross_k, *cross_v;
} fw_dec_layer;

/* Bytes of the workspace fw_decoder_step_layers needs for n_layers (0 if n_layers is out of range). The
 * caller allocates it once, zero-filled, 256-byte aligned, and passes the same workspace to every call
 * of one decoding stream; it holds control words (an epoch, an arrival count, an error flag: uint32 at
 * byte offsets 0, 4, 8), the placement fw_decoder_step_calibrate records, and the tagged hand-off
 * vectors. */
size_t fw_decoder_step_workspace_bytes(int n_layers);
int fw_decoder_step_max_layers(void);

/* Places the workspace's hand-off words: measures, for each 8 KB page of the workspace's hand-off area,
 * which half of the device (XCDs 0-3 or 4-7, each with its own I/O die) reaches it faster, and records it
 * in the workspace. Every hand-off word is kept in two copies, one on a page local to each half, and
 * each block polls the copy local to it. Call once after allocating the workspace (a few milliseconds of
 * device time, three launches on `stream`, no host synchronisation); a workspace that is never calibrated
 * gives the same results, with the copies placed without regard to locality. No counterpart in the
 * reference: it places the data of the one-launch step. */
int fw_decoder_step_calibrate(void* workspace, int64_t ws_bytes, int n_layers, hipStream_t stream);
/* 1 if the last fw_decoder_step_calibrate of this workspace measured every page (both halves' XCD pairs
 * ran), 0 if not, FW_EHIP if the workspace cannot be read. Synchronous (a 4-byte device-to-host copy). */
int fw_decoder_step_calibrated(const void* workspace);

/* The decoder layers of one token in ONE launch: replaces the per-layer op chain of the reference step
 * (custom/model.py:107-121: add_layernorm, the q/k/v, out, cross-q, cross-out, fc1, fc2 F.linear
 * calls and the two decode_attention calls per layer, whisper_kernels.cu:215-267,102-213) with the
 * arithmetic of fw_ln_gemv / fw_attention_split / fw_attn_out_gemv / fw_gemv, outputs bit-identical.
 * Starts from the embedding of token cur[0] at position state[0] (as fw_ln_gemv's embedding mode),
 * writes each layer's new K/V row at state[0], and leaves the final residual stream split as the LM
 * head takes it: h_out (residual before the last fc2 output) and x_out (that output), fp16[1280] each.
 * d_model 1280, 20 heads, FFN 5120; max_pos <= 512, enc_len <= 2048, n_layers <= 8; scale is the
 * attention scale (1/8). One block per CU, all resident at once: nothing else may run on the device
 * concurrently (no second call in flight on another stream). Every internal wait is bounded by
 * spin_limit ticks of the 100 MHz wall clock; a wait that runs out sets the workspace's error word
 * (byte offset 8) to nonzero, the launch then completes with undefined outputs, and the caller must
 * check the word and clear it. */
int fw_decoder_step_layers(const fw_dec_layer* layers, int n_layers, const int64_t* cur, const int64_t* state,
                           const void* embed, const void* pos_embed, int vocab, int max_pos, int enc_len, float scale,
                           void* h_out, void* x_out, void* workspace, int64_t ws_bytes, int64_t spin_limit,
                           hipStream_t stream);

/* The LM head of fw_decoder_step: final LayerNorm (gamma, beta, eps), the tied fp16 table w [vocab, 1280]
 * with its int8 copy wq [vocab, 1280] and meta fp32 [vocab, 2] (fw_lm_head_q8_pack), the suppress mask
 * u8 [vocab], the token list the finalize appends to (int64 [max_pos]), optionally y_out fp16[1280]
 * (NULL: not written) for the final LayerNorm output the LM head scores, optionally host_tokens (NULL:
 * not written): host memory, int64 [max_pos], coherent with the device (hipHostMallocCoherent), into
 * which every token is also stored at its index as soon as it is decoded, so a host can poll for it
 * while the launch runs; and the end-of-text ids: the launch ends after the first step whose token is
 * one of eos[0 .. n_eos), n_eos <= 4. */
typedef struct fw_dec_head {
  const void *ln_gamma, *ln_beta;
  float ln_eps;
  const void *w, *wq;
  const float* meta;
  const uint8_t* suppress;
  int64_t* tokens;
  void* y_out;
  int64_t* host_tokens;
  int n_eos;
  int64_t eos[4];
} fw_dec_head;

/* The prompt pass as ONE launch: the 4 prompt tokens prompt[0 .. 3] (int64, device) at positions
 * state[0] .. state[0] + 3 run through the decoder layers together (every phase on 4 vectors, the
 * self attention of position state[0] + z seeing the fresh K/V rows of positions state[0] .. state[0] + z,
 * all 4 K/V rows written to the caches), then the LM head, argmax and finalize on the last position
 * (replaces custom/model.py:196-207: 4 steps whose first 3 predictions are discarded). Leaves the
 * cache rows, state, cur and tokens of those 4 steps, bit for bit. The LM head applies head->suppress
 * as it is: for the first generated token pass the first step's mask (suppress plus begin-suppress ids,
 * custom/model.py:60-61,202). n_prompt == 4; same workspace, limits and residency rules as
 * fw_decoder_step. */
int fw_decoder_prompt(const fw_dec_layer* layers, int n_layers, const fw_dec_head* head, const int64_t* prompt,
                      int n_prompt, int64_t* cur, int64_t* state, const void* embed, const void* pos_embed, int vocab,
                      int max_pos, int enc_len, float scale, void* workspace, int64_t ws_bytes, int64_t spin_limit,
                      hipStream_t stream);

/* Host memory for fw_dec_head.host_tokens: `bytes` of pinned host memory that device stores reach
 * while a kernel runs (hipHostMalloc with hipHostMallocCoherent); NULL on failure. No counterpart in the
 * reference (it copies each chunk's tokens after the chunk, custom/model.py:208-215). */
void* fw_host_alloc_coherent(size_t bytes);
void fw_host_free(void* p);

/* n_steps whole decoder steps in ONE launch: each is fw_decoder_step_layers followed by the final
 * LayerNorm, the LM head with the int8 pre-pass, the argmax and the finalize (replaces n_steps calls of
 * custom/model.py:107-123, i.e. the per-layer ops above plus lm_head_argmax and argmax_finalize,
 * whisper_kernels.cu:278-298, as the 8-step graph of custom/model.py:125-141 replays them). Every
 * token is that of fw_lm_head_argmax_q8 + fw_argmax_finalize, bit for bit: tokens[state[1]] <- token,
 * state advances, cur <- token, after every step; a step takes the previous step's token and state
 * from words the finalizing block broadcasts. Same workspace, limits and residency rules as
 * fw_decoder_step_layers; 1 <= n_steps <= 1024; vocab <= 224 * (the device's CU count). */
int fw_decoder_step(const fw_dec_layer* layers, int n_layers, const fw_dec_head* head, int n_steps, int64_t* cur,
                    int64_t* state, const void* embed, const void* pos_embed, int vocab, int max_pos, int enc_len,
                    float scale, void* workspace, int64_t ws_bytes, int64_t spin_limit, hipStream_t stream);

/* Whether fw_decoder_step (prompt = 0) or fw_decoder_prompt (prompt = 1) can run these sizes on the
 * current device: FW_OK, or FW_EINVAL with the reason in fw_last_error() (too few CUs for a phase's
 * blocks, a vocabulary whose per-block LM-head share exceeds the kernel's candidate list, max_pos or
 * enc_len out of range). The launches run the same checks; a caller probes with it to choose the
 * 34-launch step instead. No counterpart in the reference (its step is separate launches). */
int fw_decoder_step_check(int n_layers, int vocab, int max_pos, int enc_len, int prompt);

/* Rows of the int8 LM-head table each block of fw_decoder_step keeps in LDS for the whole launch on the
 * current device (read from HBM once per launch; the rest of its share streams every step), or a
 * negative status. No counterpart in the reference (its LM head, whisper_kernels.cu:28-86, streams the
 * whole fp16 table every step). */
int fw_decoder_step_resident_rows(void);

/* Phase timeline of fw_decoder_step / fw_decoder_prompt, for a profiling build of the library only
 * (decode_step.hip compiled with FW_STEP_TIMELINE=1; the product build returns FW_EINVAL and 0 slots).
 * buf (device memory, NULL to stop recording) receives, for each of the first `steps` steps of every
 * later launch, each block's 100 MHz wall-clock ticks at fixed points: int64 at
 * [(step * grid + block) * slots + s], grid = min(CU count, 1024), slots from
 * fw_decoder_step_timeline_slots(). s = 0: the step starts; 1 + (l * 8 + p - 1) * 4 + k for layer
 * l < 4, phase p = 1..8 (LN1+q/k/v, self attention, out, LN2+cross q, cross attention, cross-out,
 * LN3+fc1, fc2) and k = 0 entered with its loads issued, 1 input in, 2 output stored, 3 the cross
 * attention's head combine stored / the self attention's split rounds done / a LayerNorm phase's
 * residual contributions added; 129 + k for the LM head: k = 0 arrived, 1 final LayerNorm done, 2 y
 * digits ready, 3 first two HBM batches scored, 4 resident rows scored, 5 all rows scored, 6 candidates
 * listed, 7 block maximum stored, 8 (last block) maxima gathered, 9 (last block) token broadcast;
 * 141 + k inside layer 0's self attention: k = 0 fresh row written, 1 first round's wave-0 partial,
 * 2 first round merged. Slots a block does not reach in a step read 0. No counterpart in the reference (its
 * per-kernel times come from nsys, results/run07/report.txt:414-431). Synchronous. */
int fw_decoder_step_timeline(void* buf, int64_t bytes, int steps);
int fw_decoder_step_timeline_slots(void);

/* Final residual + LayerNorm + LM head + argmax, then finalize (custom/model.py:121-123):
 * r = fp16(h + x) (x may be NULL); y = LN(r); then exactly fw_lm_head_argmax on y followed by
 * fw_argmax_finalize. best must be zero on entry and is left zero. With tokens, state and cur all
 * NULL the finalize is skipped and best holds the packed winner, as after fw_lm_head_argmax. */
int fw_lm_head_argmax_fused(const void* h, const void* x, const void* gamma, const void* beta, float eps,
                            const void* w, const uint8_t* suppress, int vocab, int hidden, uint64_t* best,
                            int64_t* tokens, int64_t* state, int64_t* cur, int max_pos, hipStream_t stream);

/* int8 copy of an LM-head table for fw_lm_head_argmax_q8 (no reference counterpart; built once per
 * weight load): per row v of w fp16[vocab, hidden], meta[2v] = s_v = max|w_v| / 127 (fp32),
 * wq[v, :] = clamp(rint(w_v / s_v), -127, 127) (int8), meta[2v + 1] = an fp32 upper bound of
 * || w_v - s_v wq[v, :] ||_2. wq int8[vocab, hidden], meta fp32[2 * vocab]. hidden == 1280. */
int fw_lm_head_q8_pack(const void* w, int vocab, int hidden, void* wq, float* meta, hipStream_t stream);

/* fw_lm_head_argmax_fused with the same arguments and the same result, bit for bit, reading the int8
 * table (wq, meta from fw_lm_head_q8_pack of this w) instead of all of w. Replaces lm_head_argmax +
 * argmax_finalize (whisper_kernels.cu:28-100, custom/model.py:121-123): each block scores its rows on
 * the int8 table with an exact integer dot, bounds every fp32 logit from both sides, and evaluates only
 * the rows that can tie or beat its best lower bound on w, with the arithmetic of fw_lm_head_argmax.
 * w, wq 16-byte aligned, meta 8-byte aligned. */
int fw_lm_head_argmax_q8(const void* h, const void* x, const void* gamma, const void* beta, float eps,
                         const void* w, const void* wq, const float* meta, const uint8_t* suppress, int vocab,
                         int hidden, uint64_t* best, int64_t* tokens, int64_t* state, int64_t* cur, int max_pos,
                         hipStream_t stream);

/* ---- log-mel front end (custom/model.py:93-98) ------------------------------------------- */

/* wave fp32[n_samples] (n_samples = 480000; already zero padded) -> out fp32[128, n_frames]
 * with n_frames = n_samples / 160: periodic Hann(400), reflect-padded centred STFT (hop 160),
 * power, filters fp32[201, 128] (Slaney), log10(max(., 1e-10)), max(x, max - 8), (x + 4) / 4.
 * out16 (may be NULL) receives fp16 of the same values, time-major [n_frames, 128].
 * ws fp32[>= fw_log_mel_ws_floats(n_samples)], 16-byte aligned. fw_log_mel = fw_log_mel_prepare
 * followed by fw_log_mel_run. */
int fw_log_mel(const float* wave, int n_samples, const float* filters, float* out, void* out16, float* ws,
               int64_t ws_floats, hipStream_t stream);
int64_t fw_log_mel_ws_floats(int n_samples);
/* audio fp32[n] in host memory (pageable) -> dev fp32[n_total], the samples followed by zeros
 * (custom/model.py:103-104). The samples pass through staging, pinned host memory of at least n
 * floats, in chunks of `chunk` samples, each chunk's copy queued on stream as soon as it is staged.
 * Returns once every copy is queued; the caller must not write staging again before they complete. */
int fw_wave_upload(const float* audio, int64_t n, float* staging, float* dev, int64_t n_total, int64_t chunk,
                   hipStream_t stream);
/* The per-filterbank part of fw_log_mel, once per workspace and filterbank: the FFT twiddle table and
 * the compacted filterbank are written to the start of ws (no reference counterpart: the reference's
 * filterbank is a constant tensor, custom/model.py:37-38). */
int fw_log_mel_prepare(const float* filters, float* ws, int64_t ws_floats, hipStream_t stream);
/* The per-clip part of fw_log_mel, on a workspace that fw_log_mel_prepare filled from the same
 * filters (custom/model.py:93-98). */
int fw_log_mel_run(const float* wave, int n_samples, const float* filters, float* out, void* out16, float* ws,
                   int64_t ws_floats, hipStream_t stream);

/* ---- encoder (HF WhisperEncoder.forward semantics in fp16; MFMA) ------------------------ */

/* out[m, n] <- epilogue(sum_k a[m, k] * w[n, k]) with fp32 accumulation on MFMA.
 * a fp16[m, lda], w fp16[n, ldw], out fp16[m, ldo], bias fp16[n], res fp16[m, ldr] (epilogues that read it).
 * k % 64 == 0, n % 128 == 0; lda, ldw, ldo, ldr multiples of 8; a, w 16-byte aligned, out, bias, res
 * 8-byte aligned. q_cols is used by FW_EPI_SCALE_Q only. */
int fw_gemm(const void* a, int lda, const void* w, int ldw, const void* bias, void* out, int ldo,
            const void* res, int ldr, int m, int n, int k, int epilogue, int q_cols, hipStream_t stream);

/* Conv1d(k=3, padding=1, stride) as an implicit GEMM over a time-major input:
 * x fp16[t_in, c_in]; wp fp16[c_out, 3 * c_in] packed as wp[o, tap * c_in + c] = weight[o, c, tap];
 * out fp16[t_out, c_out] with t_out = (t_in - 1) / stride + 1. Epilogue FW_EPI_BIAS_GELU or
 * FW_EPI_BIAS_GELU_POS (res = positions fp16[t_out, c_out]). c_in % 64 == 0. */
int fw_conv1d(const void* x, int t_in, int c_in, int stride, const void* wp, const void* bias, void* out,
              int c_out, const void* res, int epilogue, hipStream_t stream);

/* Split-k product (no reference counterpart: the encoder's fc2 Linear, transformers
 * modeling_whisper.py:405-407, computed as two k halves so that 1500 x 1280 outputs still fill the
 * CUs): part[s][m][n] <- sum over k' in [s k / 2, (s + 1) k / 2) of a[m, k'] * w[n, k'] in fp32, for
 * s < splits = 2. a fp16[m, lda], w fp16[n, ldw]; part fp32 [2][m][n]; n % 128 == 0, k % 128 == 0. */
int fw_gemm_splitk(const void* a, int lda, const void* w, int ldw, float* part, int m, int n, int k, int splits,
                   hipStream_t stream);

/* The end of a split-k product and the next LayerNorm in one launch (no reference counterpart): for
 * each row r, acc = part[0][r] + part[1][r], then h[r] <- the residual epilogue of fw_gemm with that
 * acc (epilogue FW_EPI_BIAS_RESID or FW_EPI_BIAS_RESID_CLAMP: fp16(acc + bias) added to h[r] in fp16,
 * clamped to +-(65504 - 1000) with the latter, which fp16 stores as +-64512), then
 * y[r] <- fp16(LN(h[r]) * gamma + beta) of the stored h[r], as fw_layernorm_rows.
 * part fp32 [2][rows][1280] from fw_gemm_splitk; h fp16[rows, 1280] updated in place; splits == 2. */
int fw_layernorm_rows_residual(const float* part, int splits, const void* bias, void* h, const void* gamma,
                               const void* beta, void* y, int rows, int n, float eps, int epilogue,
                               hipStream_t stream);

/* Row LayerNorm: y[r] <- fp16(LN(x[r]) * gamma + beta) for r < rows, n == 1280 (F.layer_norm on fp16). */
int fw_layernorm_rows(const void* x, const void* gamma, const void* beta, void* y, int rows, int n, float eps,
                      hipStream_t stream);

/* Element count of the transposed-V buffer `vt` of the encoder attention: heads * 64 * seq_pad,
 * seq_pad = seq rounded up to a multiple of 64 (0 for non-positive arguments). The layout inside is
 * private to this library: fill it with fw_encoder_qkv or fw_encoder_pack_vt. */
long long fw_encoder_vt_elems(int seq, int heads);

/* Encoder q/k/v projection of one layer (transformers modeling_whisper.py:309-311 with
 * custom/model.py:81-91's [q; k; v] packing): y fp16[seq, heads * 64] times w fp16[3 * heads * 64,
 * heads * 64] plus bias. q columns are scaled by 1/8 after the fp16 rounding (FW_EPI_SCALE_Q);
 * q and k go to qkv fp16[seq, 3 * heads * 64] (its v columns are left untouched); v goes to vt
 * (fw_encoder_vt_elems). heads * 64 % 128 == 0. */
int fw_encoder_qkv(const void* y, const void* w, const void* bias, void* qkv, void* vt, int seq, int heads,
                   hipStream_t stream);

/* vt from the v columns of a q/k/v projection output qkv fp16[seq, 3 * heads * 64]. */
int fw_encoder_pack_vt(const void* qkv, void* vt, int seq, int heads, hipStream_t stream);

/* Encoder self-attention (transformers modeling_whisper.py:284-358, SDPA, non-causal, scale 1: q is
 * pre-scaled): q and k from qkv fp16[seq, 3 * heads * 64] ([q | k | v] per row), v from vt;
 * out fp16[seq, heads * 64]. */
int fw_encoder_attention(const void* qkv, const void* vt, void* out, int seq, int heads, hipStream_t stream);

/* Cross K/V for all decoder layers (custom/model.py:145-146) written straight into the cache layout:
 * enc fp16[t, 1280]; w fp16[layers * 2 * 1280, 1280] rows [k_0; v_0; k_1; v_1; ...];
 * bias fp16[layers * 2 * 1280]; cross_kv fp16[layers, 2, heads, t, 64]. */
int fw_cross_kv(const void* enc, int t, const void* w, const void* bias, void* cross_kv, int layers, int heads,
                hipStream_t stream);

/* ---- seeded synthetic weights (the random-init N(mean, std) fp16 generator) -------------- */

/* dst[i] <- fp16(mean + std * z(seed, tensor_id, offset + i)); z is a counter-based standard normal
 * (splitmix64 hash + Box-Muller in explicitly rounded fp32), identical on host and device. */
int fw_synth_normal_f16(void* dst, int64_t n, int64_t offset, uint64_t seed, uint64_t tensor_id, float mean,
                        float std, hipStream_t stream);
int fw_synth_normal_f16_host(uint16_t* dst, int64_t n, int64_t offset, uint64_t seed, uint64_t tensor_id,
                             float mean, float std);

#ifdef __cplusplus
}
#endif

#endif /* FLASH_WHISPER_H_ */
