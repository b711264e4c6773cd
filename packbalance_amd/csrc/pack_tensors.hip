// Model inputs of a batch of packs, built on the device from a token store
// resident in HBM and a per-step segment table, for gfx950.
//
// Reference: packbalance/data/dataset.py:33-76 (PackedDataset.__getitem__),
// which builds the same four tensors on the host, pack by pack, from the
// memory-mapped token store (data/store.py:12-56) and then copies them to the
// device.  Here the store lives in HBM once, the host sends only
// (start, length) per document of the step's packs, and one launch writes
// input_ids, labels, position_ids and doc_ids for every pack:
//   packed (rows == 0): segment i of a pack occupies [off_i, off_i + len_i),
//       off_0 = 0, off_{i+1} = off_i + len_i; doc id i on its tokens;
//   padded (rows == R): segment i occupies row i, [i*S, i*S + len_i), and the
//       whole row carries doc id i (the reference's padded form);
// on every segment: input_ids = its tokens, labels = the next token of the
// same segment (-100 on its last token), position_ids = 0 .. len-1; every
// other position: pad_token_id, -100, 0, -1.
//
// One workgroup per (pack, block of positions).  Wave 0 turns the pack's
// segment lengths into offsets in LDS (64-lane prefix sums, chunk by chunk);
// each thread then finds the segment of a position by binary search.  Token
// reads are bounds-checked against the store (the host rejects invalid
// segments before launching; the check only keeps every access in bounds).
#include "common.hpp"

namespace pb {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxSegs = 4096;  // segments per pack (LDS offsets: 32 KB)
constexpr int kPerThread = 8;   // positions per thread in one workgroup

struct PackArgs {
  const char *store;
  int elem;  // bytes per stored token: 2, 4 or 8
  int64_t store_len;
  const int64_t *seg_start, *seg_len, *pack_seg;
  int64_t seq_len, total, rows, pad;
  int64_t *input_ids, *labels, *position_ids, *doc_ids;
};

__device__ __forceinline__ int64_t token_at(const PackArgs &a, int64_t idx, bool &ok) {
  ok = idx >= 0 && idx < a.store_len;
  if (!ok) return 0;
  if (a.elem == 4) return (int64_t) reinterpret_cast<const uint32_t *>(a.store)[idx];
  if (a.elem == 2) return (int64_t) reinterpret_cast<const uint16_t *>(a.store)[idx];
  return reinterpret_cast<const int64_t *>(a.store)[idx];
}

__global__ __launch_bounds__(kThreads) void pack_tensors_kernel(PackArgs a) {
  __shared__ int64_t off[kMaxSegs + 1];
  const int64_t p = blockIdx.y;
  const int64_t s0 = a.pack_seg[p];
  // Clamped so LDS and the output rows stay in bounds whatever the table says
  // (the host validates it; a padded pack also has at most `rows` segments).
  int64_t ns = a.pack_seg[p + 1] - s0;
  ns = ns < 0 ? 0 : ns > kMaxSegs ? kMaxSegs : ns;
  if (a.rows > 0 && ns > a.rows) ns = a.rows;
  const int nseg = (int)ns;
  const int lane = threadIdx.x & 63;
  if (a.rows == 0 && threadIdx.x < 64) {
    int64_t carry = 0;
    for (int base = 0; base < nseg; base += 64) {
      const int i = base + lane;
      int64_t v = i < nseg ? a.seg_len[s0 + i] : 0;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int64_t u = __shfl_up(v, o);
        if (lane >= o) v += u;
      }
      if (i < nseg) off[i + 1] = carry + v;
      carry += __shfl(v, 63);
    }
    if (lane == 0) off[0] = 0;
  }
  __syncthreads();
  const int64_t j0 = ((int64_t)blockIdx.x * kThreads * kPerThread) + threadIdx.x;
  int64_t *in_row = a.input_ids + p * a.total, *lb_row = a.labels + p * a.total;
  int64_t *ps_row = a.position_ids + p * a.total, *dc_row = a.doc_ids + p * a.total;
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int64_t j = j0 + (int64_t)k * kThreads;
    if (j >= a.total) break;
    int64_t tok = a.pad, lab = -100, pos = 0, doc = -1;
    int seg = -1;
    int64_t rel = 0;
    if (a.rows == 0) {
      if (nseg > 0 && j < off[nseg]) {
        // Largest i with off[i] <= j.
        int lo = 0, hi = nseg - 1;
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (off[mid] <= j) lo = mid; else hi = mid - 1;
        }
        seg = lo;
        rel = j - off[lo];
        doc = seg;
      }
    } else {
      const int64_t row = j / a.seq_len;
      if (row < nseg) {
        doc = row;
        rel = j - row * a.seq_len;
        if (rel < a.seg_len[s0 + row]) seg = (int)row;
      }
    }
    if (seg >= 0) {
      const int64_t start = a.seg_start[s0 + seg], len = a.seg_len[s0 + seg];
      bool ok;
      const int64_t t = token_at(a, start + rel, ok);
      if (ok) {
        tok = t;
        pos = rel;
        if (rel + 1 < len) {
          const int64_t t1 = token_at(a, start + rel + 1, ok);
          if (ok) lab = t1;
        }
      }
    }
    in_row[j] = tok;
    lb_row[j] = lab;
    ps_row[j] = pos;
    dc_row[j] = doc;
  }
}

}  // namespace
}  // namespace pb

extern "C" int pb_pack_tensors(const void *store, int store_elem_bytes, int64_t store_len,
                               const int64_t *seg_start, const int64_t *seg_len,
                               const int64_t *pack_seg, int64_t n_packs, int64_t max_segs,
                               int64_t seq_len, int64_t rows, int64_t pad_token_id,
                               int64_t *input_ids, int64_t *labels, int64_t *position_ids,
                               int64_t *doc_ids, void *stream) {
  using namespace pb;
  clear_error();
  PB_CHECK_ARG(store_elem_bytes == 2 || store_elem_bytes == 4 || store_elem_bytes == 8,
               "pb_pack_tensors: store elements must be 2, 4 or 8 bytes");
  PB_CHECK_ARG(n_packs >= 0 && seq_len >= 1 && rows >= 0 && store_len >= 0 && max_segs >= 0,
               "pb_pack_tensors: bad sizes");
  PB_CHECK_SUPPORTED(max_segs <= kMaxSegs, "pb_pack_tensors: more than %d segments in a pack",
                     kMaxSegs);
  PB_CHECK_SUPPORTED(n_packs < 65536, "pb_pack_tensors: at most 65535 packs per launch");
  PB_CHECK_ARG(rows == 0 || max_segs <= rows, "pb_pack_tensors: a padded pack has more segments than rows");
  if (n_packs == 0) return PB_OK;
  PB_CHECK_ARG(pack_seg && input_ids && labels && position_ids && doc_ids,
               "pb_pack_tensors: null argument");
  PB_CHECK_ARG(max_segs == 0 || (store && seg_start && seg_len), "pb_pack_tensors: null argument");
  PackArgs a;
  a.store = static_cast<const char *>(store);
  a.elem = store_elem_bytes;
  a.store_len = store_len;
  a.seg_start = seg_start;
  a.seg_len = seg_len;
  a.pack_seg = pack_seg;
  a.seq_len = seq_len;
  a.total = rows == 0 ? seq_len : rows * seq_len;
  a.rows = rows;
  a.pad = pad_token_id;
  a.input_ids = input_ids;
  a.labels = labels;
  a.position_ids = position_ids;
  a.doc_ids = doc_ids;
  const int64_t per_wg = (int64_t)kThreads * kPerThread;
  dim3 grid((unsigned)((a.total + per_wg - 1) / per_wg), (unsigned)n_packs);
  hipLaunchKernelGGL(pack_tensors_kernel, grid, dim3(kThreads), 0, as_stream(stream), a);
  return launch_status("pb_pack_tensors");
}
