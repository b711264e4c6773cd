// Shared pieces of the document-masked attention kernels (gfx950, wave64).
//
// MFMA conventions used throughout (v_mfma_f32_32x32x16_bf16, verified on the
// device): for C[32x32] += A[32x16] * B[16x32], lane l (h = l / 32) holds
//   A[row = l % 32][k = 8h .. 8h+7]       (8 bf16)
//   B[k = 8h .. 8h+7][col = l % 32]       (8 bf16)
//   C[row = 8(j/4) + 4h + j%4][col = l%32] for accumulator register j = 0..15.
// A C accumulator re-used as an MFMA operand keeps lane <-> column and puts the
// accumulator rows on the k slots: slot s of half h carries row
//   pi(h, s) = 8*(s/4) + 4h + s%4       (within a 16-row k step)
// so both operands of such a product index k through pi(h, s).
#pragma once

#include <initializer_list>

#include "common.hpp"

namespace pb {
namespace attn {

// Forward kernel tiles: query rows per workgroup, KV rows per step.
constexpr int kFwdBM = 128;
constexpr int kFwdBN = 64;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16_t mfma32(const bf16x8_t &a, const bf16x8_t &b,
                                           const f32x16_t &c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16_t zero16() {
  f32x16_t z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Row offset (within a 16-row k step) carried by k slot s of lane half h.
__device__ __forceinline__ int pi_row(int h, int s) { return 8 * (s >> 2) + 4 * h + (s & 3); }

// Eight consecutive head-dim elements of one row, zero beyond `d` (the real
// head dim) or when the row is out of range.  `vec` = 16-byte path allowed.
__device__ __forceinline__ bf16x8_t load_row8(const bf16_t *row, int d0, int d, bool valid,
                                              bool vec) {
  bf16x8_t r;
  if (valid && vec && d0 + 8 <= d) {
    u32x4 raw = *reinterpret_cast<const u32x4 *>(row + d0);
    r = *reinterpret_cast<bf16x8_t *>(&raw);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (valid && d0 + i < d) ? row[d0 + i] : (bf16_t)0.0f;
  }
  return r;
}

// Packed plan entry: tile index << 1 | FULL flag.
__device__ __forceinline__ int plan_tile(int e) { return e >> 1; }
__device__ __forceinline__ bool plan_full(int e) { return e & 1; }

// ---------------------------------------------------------------- host side
inline int check_attn_shape(const char *what, int64_t b, int64_t hq, int64_t hkv, int64_t s,
                            int64_t d, int dtype) {
  PB_CHECK_ARG(dtype == PB_BF16, "%s: only bf16 q/k/v are supported (got dtype %d)", what, dtype);
  PB_CHECK_ARG(b >= 1 && hq >= 1 && hkv >= 1 && s >= 1 && d >= 1,
               "%s: bad shape b=%lld hq=%lld hkv=%lld s=%lld d=%lld", what, (long long)b,
               (long long)hq, (long long)hkv, (long long)s, (long long)d);
  PB_CHECK_ARG(hq % hkv == 0, "%s: query heads (%lld) not a multiple of kv heads (%lld)", what,
               (long long)hq, (long long)hkv);
  PB_CHECK_SUPPORTED(d <= 128, "%s: head_dim %lld > 128 is not supported", what, (long long)d);
  PB_CHECK_SUPPORTED(s < (1LL << 30) && b * hq * s < (1LL << 40) && b * hq < (1LL << 24),
                     "%s: problem too large", what);
  return PB_OK;
}

// 16-byte global access is legal when every view is 16-byte aligned at every
// (b, h, s) row start and the head dim is a multiple of 8.
inline bool views_vectorizable(int64_t d, std::initializer_list<const pb_bhsd *> views) {
  if (d % 8) return false;
  for (const pb_bhsd *v : views) {
    if (reinterpret_cast<uintptr_t>(v->data) & 15) return false;
    if ((v->stride_b % 8) || (v->stride_h % 8) || (v->stride_s % 8)) return false;
  }
  return true;
}

// Tile sizes of the backward kernels (attn_bwd.hip).
int attn_bwd_tile(int kernel, int which);

}  // namespace attn

// Classifier shared with the block-table builder (block_tables.hip).
int classify_doc_tiles(const int64_t *doc, int64_t doc_stride, int64_t b, int64_t s, int qbs,
                       int kbs, uint8_t *cls, hipStream_t st);

}  // namespace pb
