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
#include "lds_dma.hpp"

namespace pb {
namespace attn {

// KV rows per step of the query-major kernels (forward, dQ); query rows per
// step of the KV-major kernel (dK/dV).  Each wave owns 32 rows of the other
// axis, and a workgroup has 2 or 4 waves (see AttnConfig).
constexpr int kKvStep = 64;
constexpr int kQStep = 64;

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

// Document ids of the 16 rows pi_row(hh, j), j = 0..15, of a 32-row
// sub-tile whose ids sit in LDS (16-byte aligned): four runs of four
// consecutive ids, read as 16-byte vectors before any of them is compared, so
// an element mask waits for LDS once rather than once per element.
__device__ __forceinline__ void lds_docs16(const int64_t *d, int hh, int64_t (&out)[16]) {
  typedef int64_t i64x2_t __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const i64x2_t lo = *reinterpret_cast<const i64x2_t *>(d + 8 * g + 4 * hh);
    const i64x2_t hi = *reinterpret_cast<const i64x2_t *>(d + 8 * g + 4 * hh + 2);
    out[4 * g] = lo[0];
    out[4 * g + 1] = lo[1];
    out[4 * g + 2] = hi[0];
    out[4 * g + 3] = hi[1];
  }
}

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

// MFMA operand fragment read "down the columns" of a row-major LDS tile with
// ds_read_b64_tr_b16.  That instruction works on 16-lane groups: the 16
// supplied 4-element chunks form M[16][4] and lane i of the group receives
// M[i/4 + 4e][i%4], e = 0..3 (checked on the device).  With supplying lane j
// pointing at row R + j/4, column c0 + 4(j%4), lane i receives rows R..R+3 of
// column c0 + i.  Here the fragment for lane l is column col0 + l%32 and the
// eight k slots are tile rows k0 + pi(h, s) (h = l/32): two reads, rows
// k0 + 4h .. +3 (slots 0-3) and k0 + 8 + 4h .. +3 (slots 4-7).
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

__device__ __forceinline__ bf16x8_t lds_col_frag(const bf16_t *tile, int pitch, int k0, int col0,
                                                 int lane) {
  const int j = lane & 15, g = lane >> 4, h = lane >> 5;
  const int col = col0 + 16 * (g & 1) + 4 * (j & 3);
  const int row = k0 + 4 * h + (j >> 2);
  const bf16_t *p0 = tile + row * pitch + col;
  const bf16_t *p1 = p0 + 8 * pitch;
  // C-style casts: generic -> LDS address-space casts of pointers into __shared__ tiles.
  const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(p0));
  const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(p1));
  typedef short i16x8_t __attribute__((ext_vector_type(8)));
  i16x8_t r = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return *reinterpret_cast<bf16x8_t *>(&r);
}

// Row fragment (8 consecutive columns col..col+7 of row r) of a swizzled tile.
template <int DP>
__device__ __forceinline__ bf16x8_t swz_row_frag(const char *tile, int r, int col) {
  return *reinterpret_cast<const bf16x8_t *>(tile + SwzTile<DP>::off(r, col));
}

// lds_col_frag on a swizzled tile: lane l gets column col0 + l%32 at k slots
// k0 + pi(h, s).
template <int DP>
__device__ __forceinline__ bf16x8_t swz_col_frag(const char *tile, int k0, int col0, int lane) {
  const int j = lane & 15, g = lane >> 4, h = lane >> 5;
  const int col = col0 + 16 * (g & 1) + 4 * (j & 3);
  const int row = k0 + 4 * h + (j >> 2);
  const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4_t *)(tile + SwzTile<DP>::off(row, col)));
  const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4_t *)(tile + SwzTile<DP>::off(row + 8, col)));
  typedef short i16x8_t __attribute__((ext_vector_type(8)));
  i16x8_t r = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return *reinterpret_cast<bf16x8_t *>(&r);
}

// Copy ROWS rows (kv0.., DP columns of a [S][ss] bf16 view at byte address
// `base`) into a swizzled LDS tile by LDS DMA (dma16): lane i of a
// wave-level instruction writes LDS bytes [16i, 16i+16) of its 1 KiB slice,
// so each lane fetches the global chunk that the swizzle puts there.
// `off[i]` = byte offset of that chunk within the tile (precomputed per
// thread).  The caller guarantees kv0 + ROWS <= S; the buffer bound is the
// end of row S-1.  Every thread issues exactly NDMA instructions; completion
// is tracked by vmcnt.
template <int DP, int ROWS, int NT>
struct TileDma {
  static constexpr int NDMA = ROWS * DP * 2 / 16 / NT;
  static_assert(NDMA >= 1 && ROWS * DP * 2 / 16 == NDMA * NT, "tile/thread mismatch");
  __device__ static __forceinline__ void offsets(int64_t ss, int wave, int lane, uint32_t *off) {
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      int r, c;
      SwzTile<DP>::at((i * (NT / 64) + wave) * 64 + lane, r, c);
      off[i] = (uint32_t)((r * ss + c * 8) * 2);
    }
  }
  __device__ static __forceinline__ void copy(const char *base, int64_t ss, const uint32_t *off,
                                              int kv0, int S, char *dst, int wave) {
    const char *tb = base + (int64_t)kv0 * ss * 2;
    const int64_t limit = ((int64_t)(S - 1 - kv0) * ss + DP) * 2;
    constexpr int W = NT / 64;
#pragma unroll
    for (int i = 0; i < NDMA; ++i) dma16(tb, limit, off[i], dst + (i * W + wave) * 1024);
  }
  // The same for rows kv0 .. kv0 + ROWS - 1 that all lie inside the sequence
  // (the pipelined kernels: S % 64 == 0 and tiles of whole 32-row sub-tiles),
  // so no buffer bound is needed: one 64-bit multiply-add per tile.
  __device__ static __forceinline__ void copy_in(const char *base, int64_t ss, const uint32_t *off,
                                                 int kv0, char *dst, int wave) {
    const char *tb = base + (int64_t)kv0 * ss * 2;
    constexpr int W = NT / 64;
#pragma unroll
    for (int i = 0; i < NDMA; ++i) dma16(tb, 0x7fffffff, off[i], dst + (i * W + wave) * 1024);
  }
  // The same against a resource over the whole (pack, head) view: `soff` =
  // kv0 * ss * 2 bytes (the caller keeps the view's extent below 2 GiB).
  __device__ static __forceinline__ void copy_rs(__amdgpu_buffer_rsrc_t rs, uint32_t soff,
                                                 const uint32_t *off, char *dst, int wave) {
    constexpr int W = NT / 64;
#pragma unroll
    for (int i = 0; i < NDMA; ++i) dma16_rs(rs, soff, off[i], dst + (i * W + wave) * 1024);
  }
};

// Exchange with lane ^ 32 without LDS (v_permlane32_swap): returns
// f(x, x of the partner lane) for a commutative f.
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Grid decode of the query-major kernels (forward, dQ).  Workgroup i runs on
// XCD i % 8 (each XCD has its own L2).  The G query heads that read one KV
// head's K/V tiles are placed on the same XCD, 8 workgroup ids apart, so they
// share those tiles in that XCD's L2; the groups of one (pack, KV head) follow
// each other late query tile first (the most causal work first), so the
// workgroups resident on an XCD are neighbouring query tiles of ONE pack that
// walk the same K/V tiles from its documents' starts in step (packs outer:
// cfg3 forward 1.56 -> 1.52 ms, cfg2 forward 31.2 -> 28.5 us against packs
// inner).  Within whole chunks of 8*G workgroups the map is a bijection onto
// logical ids; the tail keeps the identity map.
__device__ __forceinline__ void decode_q_major(int bid, int nqt, int B, int Hq, int Hkv, int &qt,
                                               int &b, int &h) {
  const int G = Hq / Hkv;
  const int total = nqt * B * Hq;
  const int chunk = 8 * G;
  const int full = (total / chunk) * chunk;
  int L = bid;  // logical id: group member fastest, then KV head, late-first tile, pack
  if (bid < full) {
    const int c = bid / chunk, r = bid - (bid / chunk) * chunk;
    L = (c * 8 + (r & 7)) * G + (r >> 3);
  }
  const int g = L % G;
  int t = L / G;
  const int hk = t % Hkv;
  t /= Hkv;
  qt = nqt - 1 - t % nqt;
  b = t / nqt;
  h = hk * G + g;
}

// Packed plan entry: tile index << 2 | kind, kind 1 = FULL (no element mask),
// 2 = CAUSAL (every pair with kv <= q in the tile shares a document, so the
// causal test alone is the mask), 0 = PARTIAL (document and causal tests).
__device__ __forceinline__ int plan_tile(int e) { return e >> 2; }
__device__ __forceinline__ bool plan_full(int e) { return (e & 3) == 1; }
__device__ __forceinline__ bool plan_causal(int e) { return (e & 3) == 2; }

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

// Launch shape of the three kernels for one problem size.  A workgroup of W
// waves covers 32*W rows; 4 waves amortise each staged tile over more MFMAs,
// 2 waves double the grid when the problem is small (one 2048-token pack has
// only 12 heads x 16 query tiles).  When even that leaves the dK/dV grid
// short, every query head of a GQA group gets its own workgroup and writes an
// fp32 partial that a small kernel sums (split).
//
// Forward KV split: a packed pack holds a few long documents, so the KV list
// of a late query tile can be 10-30 tiles long while the average is a third
// of that; on a small grid the longest list sets the kernel time.  When the
// grid is small, each query tile's list is cut into chunks of fwd_chunk KV
// tiles, one workgroup per chunk (fwd_splits = most chunks any list can
// need); a tile with more than one chunk leaves normalised fp32 partial
// outputs and their log-sum-exps, merged by a combine kernel.
// Kept dS (head dim 128): one block of bf16 dS per (pack, KV head, 64-row
// query tile, 64-row KV tile) at or below the diagonal, laid out
// [KV half][head of the GQA group][query half][32 KV rows][32 query slots]
// (2 KiB per 32 x 32 sub-block, G * 8 KiB per block), blocks addressed
// densely over the causal triangle: block (qt, kt) at qt (qt + 1) / 2 + kt.
// Only the plan's non-empty blocks are written and read.  Query slot s of a
// sub-block holds query row 8 ((s % 16) / 4) + 4 (s / 16) + s % 4 (the row
// order of the dK/dV kernel's dS accumulators).
constexpr int64_t kDsMaxBytes = 32LL << 30;
inline int64_t ds_tri(int64_t s) { return (s / 64) * (s / 64 + 1) / 2; }
inline int64_t ds_pair_bytes(int64_t g, int64_t s) { return ds_tri(s) * g * 8192; }
inline int64_t ds_bytes(int64_t b, int64_t hq, int64_t hkv, int64_t s) {
  return b * hkv * ds_pair_bytes(hq / hkv, s);
}

struct AttnConfig {
  int fwd_waves, dq_waves, kv_waves, split;
  int pairs;  // head dim 128 on a full grid: dK/dV by attn_bwd_dkdv_pairs on 64-row KV tiles
  // dS kept: the paired dK/dV kernel stores its bf16 dS tiles and dQ = scale * dS K
  // is a streaming pass over them (attn_bwd_dq_ds) instead of a kernel that
  // recomputes S and dP; D = rowsum(dO * O) then comes from attn_bwd_delta.
  int ds;
  int fwd_chunk, fwd_splits;  // 0 / 1: no forward KV split
  int dq_chunk, dq_splits;    // the same for the (q-major) dQ kernel
  int fwd_q_tile() const { return 32 * fwd_waves; }
  int dq_q_tile() const { return 32 * dq_waves; }
  int kv_tile() const { return 32 * kv_waves; }
};

inline AttnConfig attn_config(int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t d) {
  const int64_t kFill = 512;  // two workgroups per CU on 256 CUs
  auto tiles = [&](int rows) { return (s + rows - 1) / rows; };
  AttnConfig c;
  const bool big_q = b * hq * tiles(128) >= kFill;
  c.fwd_waves = big_q ? 4 : 2;
  c.dq_waves = big_q ? 4 : 2;
  c.kv_waves = b * hkv * tiles(128) >= kFill ? 4 : 2;
  c.split = (c.kv_waves == 2 && b * hkv * tiles(64) < kFill && hq > hkv) ? 1 : 0;
  // Head dim 128 on a full grid: two (P, dP) wave pairs per 64-row KV tile,
  // two workgroups per CU (the KV tile of the 2-wave kernels).
  c.pairs = (d == 128 && c.kv_waves == 4) ? 1 : 0;
  if (c.pairs) c.kv_waves = 2;
  c.ds = (c.pairs && (hq / hkv) % 4 == 0 && ds_pair_bytes(hq / hkv, s) < (1LL << 31) &&
          ds_bytes(b, hq, hkv, s) <= kDsMaxBytes) ? 1 : 0;
  if (c.ds) c.dq_waves = 2;  // dQ on the 64-row query tiles of the dS blocks
  // Aim for ~2048 chunk workgroups over all lists, but at least 4 KV tiles
  // each (a chunk also pays the prologue and the merge).  Measured on the
  // cfg2 step (two [2, 2048] micro-batches on two streams; attention kernel
  // time per 9 traced steps): ~4096 chunks 30.6 ms, ~2048 29.4, no split 29.6.
  auto kv_split = [&](int64_t q_rows, int &chunk_out, int &splits_out) {
    chunk_out = 0;
    splits_out = 1;
    const int64_t base = b * hq * tiles((int)q_rows), nkt = tiles(64);
    if (base >= 4 * kFill) return;
    int64_t chunk = (nkt * base + 2047) / 2048;
    if (chunk < 4) chunk = 4;
    if (chunk < nkt) {
      chunk_out = (int)chunk;
      splits_out = (int)((nkt + chunk - 1) / chunk);
    }
  };
  kv_split(c.fwd_q_tile(), c.fwd_chunk, c.fwd_splits);
  kv_split(c.dq_q_tile(), c.dq_chunk, c.dq_splits);
  return c;
}

// Workspace of pb_attn_fwd: with a KV split, the partial outputs
// [splits, b, hq, s, d] and log-sum-exps [splits, b, hq, s], fp32.
inline int64_t attn_fwd_workspace(int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t d) {
  const AttnConfig c = attn_config(b, hq, hkv, s, d);
  if (c.fwd_chunk == 0) return 0;
  const int64_t rows = (int64_t)c.fwd_splits * b * hq * s;
  return (rows * d * 4 + 255) / 256 * 256 + (rows * 4 + 255) / 256 * 256;
}

// Workspace of pb_attn_bwd: delta [b, hq, s] fp32, then (split) dK and dV
// partials [b, hq, s, d] fp32 each and a second such pair (the second halves
// of long KV lists), then (dQ KV split) dQ partials [dq_splits, b, hq, s, d]
// fp32; with kept dS (AttnConfig::ds, which excludes both splits) the dS
// blocks follow delta.
inline int64_t attn_bwd_dq_part_offset(int64_t b, int64_t hq, int64_t s, int64_t d, bool split) {
  int64_t bytes = (b * hq * s * 4 + 255) / 256 * 256;
  // split: dK and dV partials, and a second pair for lists walked in two halves
  if (split) bytes += 4 * b * hq * s * d * 4;
  return bytes;
}

inline int64_t attn_bwd_workspace(int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t d) {
  const AttnConfig c = attn_config(b, hq, hkv, s, d);
  int64_t bytes = attn_bwd_dq_part_offset(b, hq, s, d, c.split != 0);
  if (c.ds) bytes += ds_bytes(b, hq, hkv, s);  // the kept dS blocks after delta
  if (c.dq_chunk) bytes += (int64_t)c.dq_splits * b * hq * s * d * 4;
  return bytes;
}

}  // namespace attn

// Classifier shared with the block-table builder (block_tables.hip): per
// (pack, q tile, kv tile) 0 = empty, 1 = partial, 2 = full, and, only when
// causal_class is set, 3 = partial with one document for every pair kv <= q.
int classify_doc_tiles(const int64_t *doc, int64_t doc_stride, int64_t b, int64_t s, int qbs,
                       int kbs, int causal_class, uint8_t *cls, hipStream_t st);

}  // namespace pb
