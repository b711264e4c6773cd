// LDS tiles fed by LDS DMA on gfx950: the swizzled tile layout, the 16-byte
// buffer DMA that fills it, and the wait / barrier primitives of a DMA ring.
// Shared by the attention kernels and the LM-head CE GEMM.
#pragma once

#include "common.hpp"

namespace pb {

// Tiles of DP-element bf16 rows (attention K / V / Q / dO tiles, GEMM K
// slices) in LDS without padding.  Rows are packed into 256-byte lines (1, 2
// or 4 rows per line for DP = 128, 64, 32) and the 16-byte chunks of a line
// are XOR-permuted by a function of the line index.
// Measured with SQ_LDS_BANK_CONFLICT on gfx950, this layout is conflict-free
// both for ds_read_b128 row fragments (32 consecutive rows, one chunk each)
// and for the ds_read_b64_tr_b16 column fragments of lds_col_frag (8 rows x 4
// chunks per wave); a padded row pitch serves only one of the two (pitch
// DP+8 costs 2.7 conflict cycles per transposing read).
template <int DP>
struct SwzTile {
  static constexpr int CPR = DP / 8;   // 16-byte chunks per row
  static constexpr int RPL = 16 / CPR;  // rows per 256-byte line
  static constexpr int BYTES = 64 * DP * 2;  // a 64-row tile
  static_assert(DP == 32 || DP == 64 || DP == 128, "row width");
  __device__ static __forceinline__ int xmask(int line) {
    if constexpr (CPR == 16) return ((line & 3) << 2) | ((line >> 2) & 3);
    else if constexpr (CPR == 8) return ((line & 1) << 2) | ((line >> 1) & 3);
    else return line & 3;
  }
  // Byte offset of element `col` (a multiple of 4) of row r.
  __device__ static __forceinline__ int off(int r, int col) {
    const int line = r / RPL;
    return ((line * 16 + (r % RPL) * CPR + ((col >> 3) ^ xmask(line))) << 4) + ((col & 7) << 1);
  }
  // Row r and chunk c (8 elements) held by LDS chunk p of the tile.
  __device__ static __forceinline__ void at(int p, int &r, int &c) {
    const int line = p >> 4, slot = p & 15;
    r = line * RPL + slot / CPR;
    c = (slot % CPR) ^ xmask(line);
  }
};

// Raw-buffer resource word 3 on gfx9-family parts (32-bit data, no swizzle).
constexpr int kBufWord3 = 0x00020000;

// LDS DMA of 16 bytes per active lane: lane i copies bytes [voff, voff + 16)
// after `base` (wave-uniform) to LDS bytes [16i, 16i + 16) of `dst`.  Issued
// as a raw buffer load with num_records = `limit` bytes (reads past it return
// zeros instead of faulting).  The compiler counts buffer LDS loads in vmcnt
// only; a FLAT global_load_lds in flight makes it wait for every outstanding
// LDS read (lgkmcnt(0)) wherever it waits for one.
__device__ __forceinline__ void dma16(const void *base, int64_t limit, uint32_t voff, void *dst) {
  const int lim = (int)(limit < 0x7fffffff ? limit : 0x7fffffff);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, lim, kBufWord3);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)dst, 16,
                                           voff, 0, 0, 0);
}

// The same DMA against a buffer resource built once (buf_rsrc) and a
// wave-uniform byte offset `soff` (the instruction's scalar offset), so a
// loop that walks tiles of one buffer pays one scalar add per tile instead of
// rebuilding a 64-bit base and its resource for every instruction.  The
// caller keeps soff + voff + 16 within the resource's `limit` bytes.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *base, int64_t limit) {
  const int lim = (int)(limit < 0x7fffffff ? limit : 0x7fffffff);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, lim, kBufWord3);
}

__device__ __forceinline__ void dma16_rs(__amdgpu_buffer_rsrc_t rs, uint32_t soff, uint32_t voff,
                                         void *dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)dst, 16,
                                           voff, soff, 0, 0);
}

// dma16_rs for data read exactly once: the non-temporal cache policy (nt)
// marks the lines for early eviction, so a stream does not push re-used
// tiles out of L2.
__device__ __forceinline__ void dma16_rs_nt(__amdgpu_buffer_rsrc_t rs, uint32_t soff,
                                            uint32_t voff, void *dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)dst, 16,
                                           voff, soff, 0, 2);
}

// s_waitcnt vmcnt(N) with expcnt / lgkmcnt left alone: all but the N most
// recent vector-memory operations (loads, LDS DMA) of this wave have landed.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier without __syncthreads' memory fence: the fence would
// wait for every outstanding vector-memory operation (vmcnt(0)), including
// LDS DMA deliberately left in flight.  The caller waits for the DMA it needs
// (wait_vmcnt) first; the empty asm statements keep the compiler from moving
// memory accesses across the barrier.
__device__ __forceinline__ void block_sync_nofence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace pb
