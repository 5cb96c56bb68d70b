// Shared pieces of the LDS-staged MFMA kernels (encoder GEMM and encoder attention) for gfx950:
// the 16-byte-chunk XOR swizzle of 128-byte LDS rows, direct global-to-LDS copies, explicit vmcnt
// waits for a ring of copy stages, and the key order of the attention's transposed V.
#pragma once
#include "fw_common.h"

namespace fw {

// Chunk c of LDS row r (8 x 16-byte chunks per row) lives in slot c ^ ((r >> 1) & 7). An MFMA
// operand read has lane i on row r0 + i; with 64 four-byte banks (256 bytes) a 16-lane group then
// covers every (r & 1, slot) pair once, i.e. all 64 banks. The row-only XOR (c ^ (r & 7), shift 0)
// put rows r and r + 8 of a group on the same banks; the shift took the 1280-column encoder GEMM
// (K = 5120) from 43 to 36 us and the q/k/v projection from 30 to 28 us on MI355X.
#ifndef FW_SWZ_SHIFT
#define FW_SWZ_SHIFT 1
#endif
// Any shift gives a permutation of a row's 8 chunks (so every shift is correct); it sets only which
// rows share banks.
static_assert(FW_SWZ_SHIFT >= 0 && FW_SWZ_SHIFT <= 4, "FW_SWZ_SHIFT: 0..4");
__device__ __forceinline__ int swz_slot(int row, int chunk) { return chunk ^ ((row >> FW_SWZ_SHIFT) & 7); }
__device__ __forceinline__ int swz(int row, int chunk) { return row * 8 + swz_slot(row, chunk); }

// global_load_lds_dwordx4 writes one 16-byte chunk per lane straight into LDS at M0 + 16 * lane, so
// a wave instruction fills 1 KB = 8 rows of 128 bytes. The XOR swizzle is applied on the source
// side: lane l fills LDS row r0 + l / 8, slot l % 8, so it fetches chunk swz_slot(row, l % 8).
// The copies are issued from inline assembly: the compiler then does not guard every LDS read with
// a wait for all outstanding copies, and the pipeline depth is set by the explicit vmcnt waits.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(lds_base) : "memory", "m0");
}
// The same copy from a wave-uniform base (scalar registers) plus a 32-bit per-lane byte offset. A
// loop that walks the base (one k stage after another) then needs no per-copy address arithmetic in
// the vector unit: the offsets stay in registers and only the scalar base moves.
__device__ __forceinline__ void dma16_s(uint32_t voff, const void* sbase, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_base)
               : "memory", "m0");
}
#pragma clang diagnostic pop

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ void barrier_only() { asm volatile("s_barrier" ::: "memory"); }

// Waits until only the copies of the `ahead` most recently issued stages may still be in flight.
template <int kPer, int A>
__device__ __forceinline__ void wait_stages_ahead(int ahead) {
  if constexpr (A == 0) {
    wait_vmcnt<0>();
  } else {
    if (ahead >= A) wait_vmcnt<A * kPer>();
    else wait_stages_ahead<kPer, A - 1>(ahead);
  }
}

// Workgroup barrier for LDS hand-off only: waits for this wave's LDS traffic, not for its global
// loads (__syncthreads would also drain the prefetches that are meant to stay in flight). The
// lgkmcnt(0) wait goes through the builtin (encoding: vmcnt 63, expcnt 7, lgkmcnt 0) so the compiler
// knows every earlier LDS read has completed and adds no waits of its own for them afterwards; the
// barrier itself stays an asm statement with a memory clobber so no LDS access moves across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);
  asm volatile("s_barrier" ::: "memory");
}

// Keys per transposed-V row: seq rounded up to whole 64-key attention tiles.
__host__ __device__ constexpr int vt_pad(int seq) { return (seq + 63) / 64 * 64; }

// Position of key t in the transposed-V layout of the encoder attention (an involution: swaps bits 2
// and 3 of t, so the 8 keys an MFMA lane pairs with P^T are one contiguous 16-byte chunk).
__device__ __forceinline__ int vt_pos(int t) { return (t & ~12) | ((t & 4) << 1) | ((t & 8) >> 1); }

}  // namespace fw
