// Document-masked causal GQA attention in fp32 on the fp32 matrix cores
// (gfx950 v_mfma_f32_32x32x2_f32: fp32 operands, fp32 accumulation).
//
// The path for fp32 q/k/v: without autocast the reference's FlexAttention
// computes in fp32 (packbalance/model/attention.py:116-122 on fp32 tensors),
// while the bf16 kernels (attn_fwd.hip / attn_bwd.hip) round operands to bf16.
// Same mask and conventions as those kernels: allowed(i, j) = doc[i] == doc[j]
// && j <= i (padding -1 is one more document, as FlexAttention's mask_mod),
// query head h reads KV head h / (Hq / Hkv), lse in the log2 domain
// (log2 sum_j exp2(scale log2(e) q.k)).
//
// Tiles as in the bf16 kernels, with fp32 operands read one float per lane
// and MFMA (k = 2 per instruction):
//   forward / dQ  one workgroup per (pack, query head, 128 query rows), wave w
//                 owning 32 query rows with its Q (and dO) row in registers;
//                 S^T = K Q^T per 32-row KV sub-tile (lane <-> query column),
//                 then O^T += V^T P^T (forward) or dQ^T += K^T dS^T (dQ), with
//                 P^T / dS^T taken straight from the accumulators as the B
//                 operand (register r of lane half h is KV row crow(h, r), the
//                 same row the A operand of that lane reads).  The dQ kernel
//                 also forms delta = rowsum(dO * O) for the dK/dV kernel.
//   dK / dV       one workgroup per (pack, KV head, 128 KV rows), wave w owning
//                 32 KV rows with K and V in registers; it walks every query
//                 head of the GQA group and every 32-row query sub-tile at or
//                 after its rows: S = Q K^T and dP = dO V^T (lane <-> KV
//                 column), then dV^T += dO^T P and dK^T += Q^T dS.
// K / V (or Q / dO) sub-tiles pass through LDS, staged in registers one
// sub-tile ahead, in the layout each product reads as 16-byte vectors: row
// split (a row's even then odd columns) for the A operand of S-type products,
// transposed for that of PV-type products; the head dim is padded to DP (32,
// 64 or 128) with zeros.  A workgroup first lists the sub-tiles that hold an
// allowed pair for any of its rows (its rows' document runs against every
// position of the other axis, visit_list) and loads only those; a wave then
// skips a listed sub-tile whose 32 x 32 pairs hold none for its own rows.  So
// the work follows the documents, and nothing past the causal bound is read.
#include <type_traits>

#include "attn_common.hpp"

namespace pb {
namespace attn32 {

struct View {
  float *p;
  int64_t sb, sh, ss;
  __device__ __forceinline__ float *row(int b, int h, int s) const {
    return p + b * sb + h * sh + (int64_t)s * ss;
  }
};

struct Args {
  View q, k, v, o, dout, dq, dk, dv;
  float *lse;    // [B][Hq][S], log2 domain
  float *delta;  // [B][Hq][S], rowsum(dO * O) (backward)
  const int64_t *doc;
  int64_t doc_sb;
  int B, Hq, Hkv, S, D;
  float scale;  // softmax scale
  int vec;      // K / V / Q / dO rows may be read as float4 (D % 4 == 0, 16-byte aligned rows)
  // dK/dV step chunking on small grids: a KV tile's steps (heads x listed
  // query sub-tiles) are cut into at most nsplit chunks of at least
  // kMinChunk steps, one workgroup each (chunk index = blockIdx.x / tiles).  A
  // tile with more than one chunk leaves per-chunk fp32 dK and dV rows (D
  // floats) at part / part2 (+ c * pstride) that attn_f32_sum_chunks adds up;
  // nch[tile] = its chunk count.
  int nsplit;
  int *nch;
  float *part, *part2;
  int64_t pstride;
};

constexpr int kMinChunk = 4;

// Chunk c of a list of n >= 1 entries: [i0, i1) and the tile's chunk count.
__device__ __forceinline__ void chunk_of(int n, int nsplit, int c, int &i0, int &i1, int &nch) {
  int ch = (n + nsplit - 1) / nsplit;
  if (ch < kMinChunk) ch = kMinChunk;
  nch = (n + ch - 1) / ch;
  i0 = c * ch;
  i1 = min(n, i0 + ch);
}

using attn::f32x16_t;
using attn::zero16;

constexpr int kWaves = 4;           // waves per workgroup
constexpr int kRows = 32 * kWaves;  // rows per workgroup (query rows, or KV rows for dK/dV)

__device__ __forceinline__ f32x16_t mfma(float a, float b, const f32x16_t &c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Row of a 32 x 32 MFMA accumulator held in register r by lane half h.
__device__ __forceinline__ int crow(int h, int r) { return 8 * (r >> 2) + 4 * h + (r & 3); }

__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32); }

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Lane (l32, h)'s A operands of an S-type product from a row-split tile:
// k-steps 4q .. 4q + 3 (columns 2k + h of row l32).
template <int DP>
__device__ __forceinline__ f32x4_t rs4(const float *rs, int l32, int hh, int q) {
  return *reinterpret_cast<const f32x4_t *>(rs + l32 * (DP + 4) + hh * (DP / 2) + 4 * q);
}
// Lane (l32, h)'s A operands of a PV-type product from a transposed tile: the
// values of column 32 db + l32 at rows crow(h, 4g .. 4g + 3).
__device__ __forceinline__ f32x4_t tr4(const float *tr, int db, int l32, int hh, int g) {
  return *reinterpret_cast<const f32x4_t *>(tr + (32 * db + l32) * 36 + 8 * g + 4 * hh);
}

// A [32][DP] fp32 sub-tile (rows r0 .. r0 + 31 of one (pack, head) view,
// columns past D and rows past S zero), staged in registers by the
// workgroup's 256 threads and stored to LDS at pitch DP + 1.
template <int DP>
struct Tile {
  static constexpr int N = 32 * DP / (64 * kWaves);  // floats per thread
  float v[N];
  __device__ __forceinline__ void load(const View &t, int b, int hh, int r0, int S, int D,
                                       bool vec) {
    const int tid = threadIdx.x;
    if (vec) {  // 16-byte chunks (D % 4 == 0)
#pragma unroll
      for (int i = 0; i < N / 4; ++i) {
        const int e = tid + 64 * kWaves * i;
        const int row = e / (DP / 4), col = (e % (DP / 4)) * 4;
        float4 x = {0.f, 0.f, 0.f, 0.f};
        if (r0 + row < S && col < D) x = *reinterpret_cast<const float4 *>(t.row(b, hh, r0 + row) + col);
        v[4 * i] = x.x;
        v[4 * i + 1] = x.y;
        v[4 * i + 2] = x.z;
        v[4 * i + 3] = x.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int e = tid + 64 * kWaves * i;
        const int row = e / DP, col = e % DP;
        v[i] = (r0 + row < S && col < D) ? t.row(b, hh, r0 + row)[col] : 0.f;
      }
    }
  }
  // (row, col) of the i-th value this thread holds.
  __device__ __forceinline__ void at(int i, bool vec, int &row, int &col) const {
    const int tid = threadIdx.x;
    if (vec) {
      const int e = tid + 64 * kWaves * (i / 4);
      row = e / (DP / 4);
      col = (e % (DP / 4)) * 4 + i % 4;
    } else {
      const int e = tid + 64 * kWaves * i;
      row = e / DP;
      col = e % DP;
    }
  }
  // Row-split layout (the A operand of S-type products, A[row][k = 2j + h]):
  // row r at r * kRsPitch, its even columns then its odd ones, so lane half h
  // reads its DP / 2 values of a row as contiguous 16-byte vectors.
  static constexpr int kRsPitch = DP + 4;
  static constexpr int kRsFloats = 32 * kRsPitch;
  __device__ __forceinline__ void store_rs(float *lds, bool vec) const {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      int row, col;
      at(i, vec, row, col);
      lds[row * kRsPitch + (col & 1) * (DP / 2) + (col >> 1)] = v[i];
    }
  }
  // Transposed layout (the A operand of PV-type products, A[d][k = row]):
  // column c at c * kTrPitch, so a lane reads the rows crow(h, 4g .. 4g + 3)
  // of its column as one 16-byte vector.
  static constexpr int kTrPitch = 36;
  static constexpr int kTrFloats = DP * kTrPitch;
  __device__ __forceinline__ void store_tr(float *lds, bool vec) const {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      int row, col;
      at(i, vec, row, col);
      lds[col * kTrPitch + row] = v[i];
    }
  }
};

// Sub-tiles of the other axis that hold at least one allowed pair with the
// workgroup's own rows [r0, r0 + kRows): the own rows' documents as runs, then
// every other-axis position p in [lo, hi) against them -- q-major kernels (own
// rows are queries, p a KV position) need doc[p] equal to a run's and p at or
// before its last query; the KV-major kernel (own rows are KV rows, p a query)
// needs doc[p] equal and p at or after the run's first KV row.  The 32-row
// sub-tiles holding such a p are listed in ascending order (absolute indices);
// returns their count, or -1 when the range has more than kMaxList sub-tiles
// (the caller then visits every one).  Called by the whole workgroup.
constexpr int kMaxList = 1024;

struct Visit {
  int64_t rdoc[kRows];
  int rlo[kRows], rhi[kRows];
  unsigned char flag[kMaxList];
  int list[kMaxList];
  int nrun, cnt;
};

template <bool QMAJOR>
__device__ int visit_list(Visit &vs, const int64_t *docb, int S, int r0, int lo, int hi) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t0 = lo / 32, nt = (hi + 31) / 32 - t0;  // lo is a multiple of 32
  if (nt > kMaxList) return -1;                       // uniform
  const int own_end = min(S, r0 + kRows);
  int64_t d = 0;
  const bool valid = tid < kRows && r0 + tid < S;
  if (tid < kRows) {
    d = valid ? docb[r0 + tid] : 0;
    vs.rdoc[tid] = d;  // own documents first; the runs overwrite them below
  }
  for (int i = tid; i < nt; i += 64 * kWaves) vs.flag[i] = 0;
  __syncthreads();
  const bool start = valid && (tid == 0 || vs.rdoc[tid - 1] != d);
  const uint64_t bal = __builtin_amdgcn_ballot_w64(start);
  if (wave == 0 && lane == 0) vs.cnt = __popcll(bal);  // runs starting in wave 0
  __syncthreads();
  if (start) {
    const int id = (wave == 1 ? vs.cnt : 0) + __popcll(bal & ((1ull << lane) - 1));
    vs.rdoc[id] = d;
    vs.rlo[id] = r0 + tid;
  }
  if (wave == 1 && lane == 0) vs.nrun = vs.cnt + __popcll(bal);
  __syncthreads();
  const int nrun = vs.nrun;
  for (int j = tid; j < nrun; j += 64 * kWaves)
    vs.rhi[j] = (j + 1 < nrun ? vs.rlo[j + 1] : own_end) - 1;
  __syncthreads();
  for (int p = lo + tid; p < hi; p += 64 * kWaves) {
    const int64_t dp = docb[p];
    bool ok = false;
    for (int j = 0; j < nrun; ++j)
      ok |= dp == vs.rdoc[j] && (QMAJOR ? p <= vs.rhi[j] : p >= vs.rlo[j]);
    if (ok) vs.flag[p / 32 - t0] = 1;
  }
  __syncthreads();
  if (wave == 0) {
    int n = 0;
    for (int base = 0; base < nt; base += 64) {
      const bool f = base + lane < nt && vs.flag[base + lane];
      const uint64_t b = __builtin_amdgcn_ballot_w64(f);
      if (f) vs.list[n + __popcll(b & ((1ull << lane) - 1))] = t0 + base + lane;
      n += __popcll(b);
    }
    if (lane == 0) vs.cnt = n;
  }
  __syncthreads();
  return vs.cnt;
}

// ---------------------------------------------------------------- forward
// Head dim 128 (Q, O^T, the staged tiles and the K column reads hoisted ahead of
// the S^T chain: ~300 registers) runs one wave per SIMD.
template <int DP>
__global__ __launch_bounds__(64 * kWaves)
__attribute__((amdgpu_waves_per_eu(DP == 128 ? 1 : 2, DP == 128 ? 1 : 2)))
void attn_fwd_f32(Args a) {
  constexpr int NS = DP / 2, NDB = DP / 32;
  __shared__ __align__(16) float Ks[Tile<DP>::kRsFloats], Vs[Tile<DP>::kTrFloats];
  __shared__ int64_t kd[32];
  __shared__ Visit vis;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hh = lane >> 5, l32 = lane & 31;
  const int S = a.S, D = a.D;
  const int nqt = (S + kRows - 1) / kRows;
  const int qt = nqt - 1 - (int)(blockIdx.x % nqt);  // late query tiles (longest walks) first
  const int bh = (int)(blockIdx.x / nqt), h = bh % a.Hq, b = bh / a.Hq;
  const int hk = h / (a.Hq / a.Hkv);
  const bool vec = a.vec != 0;
  const int64_t *docb = a.doc + b * a.doc_sb;
  const float sl2 = a.scale * kLog2e;

  const int qi = qt * kRows + wave * 32 + l32;
  const bool qv = qi < S;
  const int64_t qdoc = docb[qv ? qi : S - 1];
  float qf[NS];  // B operand of S^T = K Q^T: Q[qi][2k + hh], scaled into the log2 domain
  {
    const float *qr = a.q.row(b, h, qv ? qi : 0);
#pragma unroll
    for (int k = 0; k < NS; ++k) qf[k] = (qv && 2 * k + hh < D) ? qr[2 * k + hh] * sl2 : 0.f;
  }
  f32x16_t oacc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) oacc[i] = zero16();
  float m = -INFINITY, l = 0.f;

  // KV sub-tiles up to the causal bound that hold an allowed pair for some row
  // of the workgroup.
  const int kv_end = min(S, (qt + 1) * kRows);
  const int nl = visit_list<true>(vis, docb, S, qt * kRows, 0, kv_end);
  const int nst = nl >= 0 ? nl : (kv_end + 31) / 32;
  auto tile_of = [&](int i) { return nl >= 0 ? vis.list[i] : i; };
  Tile<DP> tk, tv;
  int64_t dnext = 0;
  auto fetch = [&](int st) {
    tk.load(a.k, b, hk, 32 * st, S, D, vec);
    tv.load(a.v, b, hk, 32 * st, S, D, vec);
    if (tid < 32) dnext = 32 * st + tid < S ? docb[32 * st + tid] : 0;
  };
  fetch(tile_of(0));  // nst >= 1: row qi always sees itself
  for (int i = 0; i < nst; ++i) {
    __syncthreads();  // every wave is done with the previous sub-tile
    tk.store_rs(Ks, vec);
    tv.store_tr(Vs, vec);
    if (tid < 32) kd[tid] = dnext;
    __syncthreads();
    const int kv0 = 32 * tile_of(i);
    if (i + 1 < nst) fetch(tile_of(i + 1));
    unsigned okm = 0;  // bit r: pair (KV row crow(hh, r), query qi) allowed
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kv = kv0 + crow(hh, r);
      okm |= (unsigned)(qv && kv <= qi && kd[crow(hh, r)] == qdoc) << r;
    }
    if (__builtin_amdgcn_ballot_w64(okm != 0) == 0) continue;  // uniform over the wave
    f32x16_t sacc = zero16();
#pragma unroll
    for (int q4 = 0; q4 < NS / 4; ++q4)
      if (8 * q4 < D) {
        const f32x4_t ka = rs4<DP>(Ks, l32, hh, q4);
#pragma unroll
        for (int x = 0; x < 4; ++x) sacc = mfma(ka[x], qf[4 * q4 + x], sacc);
      }
    float mloc = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sacc[r] = (okm >> r) & 1 ? sacc[r] : -INFINITY;
      mloc = fmaxf(mloc, sacc[r]);
    }
    mloc = fmaxf(mloc, xor32(mloc));  // the other lane half holds the other 16 KV rows
    const float mn = fmaxf(m, mloc);
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float alpha = fast_exp2(m - mu);  // 0 while m is -inf
    m = mn;
    l *= alpha;
#pragma unroll
    for (int db = 0; db < NDB; ++db) oacc[db] *= alpha;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sacc[r] = fast_exp2(sacc[r] - mu);
      l += sacc[r];
    }
    // O^T += V^T P^T: step r pairs KV rows crow(0, r) and crow(1, r) (k = lane half).
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      if (32 * db < D) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4_t va = tr4(Vs, db, l32, hh, g);
#pragma unroll
          for (int x = 0; x < 4; ++x) oacc[db] = mfma(va[x], sacc[4 * g + x], oacc[db]);
        }
      }
  }
  const float lt = l + xor32(l);
  if (!qv) return;
  const float inv = 1.0f / lt;  // lt >= 1: row qi always sees itself
  float *orow = a.o.row(b, h, qi);
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 32 * db + crow(hh, r);
      if (d < D) orow[d] = oacc[db][r] * inv;
    }
  if (hh == 0) a.lse[(int64_t)bh * S + qi] = m + fast_log2(lt);
}

// ---------------------------------------------------------------- dQ (+ delta)
// Head dims 64 and 128 keep Q, dO, dQ^T and the staged tiles at one wave per
// SIMD (head dim 64 spills at two).
template <int DP>
__global__ __launch_bounds__(64 * kWaves)
__attribute__((amdgpu_waves_per_eu(DP >= 64 ? 1 : 2, DP >= 64 ? 1 : 2)))
void attn_bwd_dq_f32(Args a) {
  constexpr int NS = DP / 2, NDB = DP / 32;
  // K row-split (S^T) and transposed (dQ^T), V row-split (dP^T).
  __shared__ __align__(16) float Ks[Tile<DP>::kRsFloats], Kt[Tile<DP>::kTrFloats];
  __shared__ __align__(16) float Vs[Tile<DP>::kRsFloats];
  __shared__ int64_t kd[32];
  __shared__ Visit vis;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hh = lane >> 5, l32 = lane & 31;
  const int S = a.S, D = a.D;
  const int nqt = (S + kRows - 1) / kRows;
  const int qt = nqt - 1 - (int)(blockIdx.x % nqt);
  const int bh = (int)(blockIdx.x / nqt), h = bh % a.Hq, b = bh / a.Hq;
  const int hk = h / (a.Hq / a.Hkv);
  const bool vec = a.vec != 0;
  const int64_t *docb = a.doc + b * a.doc_sb;
  const float sl2 = a.scale * kLog2e;

  const int qi = qt * kRows + wave * 32 + l32;
  const bool qv = qi < S;
  const int64_t qdoc = docb[qv ? qi : S - 1];
  float qf[NS], gf[NS];  // Q (log2-scaled) and dO at columns 2k + hh
  float dl = 0.f;
  {
    const float *qr = a.q.row(b, h, qv ? qi : 0), *gr = a.dout.row(b, h, qv ? qi : 0);
    const float *orow = a.o.row(b, h, qv ? qi : 0);
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      const bool in = qv && 2 * k + hh < D;
      qf[k] = in ? qr[2 * k + hh] * sl2 : 0.f;
      gf[k] = in ? gr[2 * k + hh] : 0.f;
      dl = in ? fmaf(gf[k], orow[2 * k + hh], dl) : dl;
    }
  }
  dl += xor32(dl);  // delta_i = rowsum(dO_i * O_i)
  const int64_t ri = ((int64_t)b * a.Hq + h) * S + (qv ? qi : 0);
  if (qv && hh == 0) a.delta[ri] = dl;
  const float lse = qv ? a.lse[ri] : 0.f;
  f32x16_t dqacc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) dqacc[i] = zero16();

  // KV sub-tiles up to the causal bound that hold an allowed pair for some row
  // of the workgroup.
  const int kv_end = min(S, (qt + 1) * kRows);
  const int nl = visit_list<true>(vis, docb, S, qt * kRows, 0, kv_end);
  const int nst = nl >= 0 ? nl : (kv_end + 31) / 32;
  auto tile_of = [&](int i) { return nl >= 0 ? vis.list[i] : i; };
  Tile<DP> tk, tv;
  int64_t dnext = 0;
  auto fetch = [&](int st) {
    tk.load(a.k, b, hk, 32 * st, S, D, vec);
    tv.load(a.v, b, hk, 32 * st, S, D, vec);
    if (tid < 32) dnext = 32 * st + tid < S ? docb[32 * st + tid] : 0;
  };
  fetch(tile_of(0));  // nst >= 1: row qi always sees itself
  for (int i = 0; i < nst; ++i) {
    __syncthreads();  // every wave is done with the previous sub-tile
    tk.store_rs(Ks, vec);
    tk.store_tr(Kt, vec);
    tv.store_rs(Vs, vec);
    if (tid < 32) kd[tid] = dnext;
    __syncthreads();
    const int kv0 = 32 * tile_of(i);
    if (i + 1 < nst) fetch(tile_of(i + 1));
    unsigned okm = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kv = kv0 + crow(hh, r);
      okm |= (unsigned)(qv && kv <= qi && kd[crow(hh, r)] == qdoc) << r;
    }
    if (__builtin_amdgcn_ballot_w64(okm != 0) == 0) continue;
    f32x16_t sacc = zero16(), pacc = zero16();
#pragma unroll
    for (int q4 = 0; q4 < NS / 4; ++q4)
      if (8 * q4 < D) {
        const f32x4_t ka = rs4<DP>(Ks, l32, hh, q4), va = rs4<DP>(Vs, l32, hh, q4);
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          sacc = mfma(ka[x], qf[4 * q4 + x], sacc);  // S^T = K Q^T
          pacc = mfma(va[x], gf[4 * q4 + x], pacc);  // dP^T = V dO^T
        }
      }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = (okm >> r) & 1 ? fast_exp2(sacc[r] - lse) : 0.f;
      sacc[r] = p * (pacc[r] - dl);  // dS^T
    }
    // dQ^T += K^T dS^T
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      if (32 * db < D) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4_t ka = tr4(Kt, db, l32, hh, g);
#pragma unroll
          for (int x = 0; x < 4; ++x) dqacc[db] = mfma(ka[x], sacc[4 * g + x], dqacc[db]);
        }
      }
  }
  if (!qv) return;
  float *dqr = a.dq.row(b, h, qi);
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 32 * db + crow(hh, r);
      if (d < D) dqr[d] = dqacc[db][r] * a.scale;
    }
}

// ---------------------------------------------------------------- dK, dV
// Head dims 64 and 128 keep K, V, dK^T, dV^T and the staged tiles at one wave
// per SIMD (head dim 64 spills at two).
template <int DP>
__global__ __launch_bounds__(64 * kWaves)
__attribute__((amdgpu_waves_per_eu(DP >= 64 ? 1 : 2, DP >= 64 ? 1 : 2)))
void attn_bwd_dkdv_f32(Args a) {
  constexpr int NS = DP / 2, NDB = DP / 32;
  // Q and dO row-split (S, dP) and transposed (dK^T, dV^T).
  __shared__ __align__(16) float Qs[Tile<DP>::kRsFloats], Gs[Tile<DP>::kRsFloats];
  __shared__ __align__(16) float Qt[Tile<DP>::kTrFloats], Gt[Tile<DP>::kTrFloats];
  __shared__ int64_t qd[32];
  __shared__ float ls[32], dls[32];
  __shared__ Visit vis;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hh = lane >> 5, l32 = lane & 31;
  const int S = a.S, D = a.D;
  const int G = a.Hq / a.Hkv;
  const int nkt = (S + kRows - 1) / kRows;
  const int tiles = a.B * a.Hkv * nkt;
  const int chunk = (int)blockIdx.x / tiles, tb = (int)blockIdx.x - chunk * tiles;
  const int kt = tb % nkt;
  const int bh = tb / nkt, hk = bh % a.Hkv, b = bh / a.Hkv;
  const bool vec = a.vec != 0;
  const int64_t *docb = a.doc + b * a.doc_sb;
  const float sl2 = a.scale * kLog2e;

  const int kv = kt * kRows + wave * 32 + l32;
  const bool kvv = kv < S;
  const int64_t kvdoc = docb[kvv ? kv : S - 1];
  float kf[NS], vf[NS];  // B operands of S = Q K^T (K log2-scaled) and dP = dO V^T
  {
    const float *kr = a.k.row(b, hk, kvv ? kv : 0), *vr = a.v.row(b, hk, kvv ? kv : 0);
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      const bool in = kvv && 2 * k + hh < D;
      kf[k] = in ? kr[2 * k + hh] * sl2 : 0.f;
      vf[k] = in ? vr[2 * k + hh] : 0.f;
    }
  }
  f32x16_t dkacc[NDB], dvacc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) {
    dkacc[i] = zero16();
    dvacc[i] = zero16();
  }

  // Steps t = (query head g of the group, listed 32-row query sub-tile): the
  // sub-tiles at or after the workgroup's first KV row that hold an allowed
  // pair for some of its rows (the same for every head of the group).
  const int st0 = (kt * kRows) / 32;
  const int nl = visit_list<false>(vis, docb, S, kt * kRows, kt * kRows, S);
  const int nq = nl >= 0 ? nl : (S + 31) / 32 - st0;
  auto tile_of = [&](int i) { return nl >= 0 ? vis.list[i] : st0 + i; };
  const int T = G * nq;
  int i0, i1, nch;  // this workgroup's steps [i0, i1) of the T
  chunk_of(T, a.nsplit, chunk, i0, i1, nch);
  if (i0 >= i1) return;  // uniform: an empty chunk slot
  if (chunk == 0 && tid == 0 && a.nsplit > 1) a.nch[bh * nkt + kt] = nch;
  Tile<DP> tq, tg;
  int64_t dnext = 0;
  float lnext = 0.f;
  auto fetch = [&](int t) {
    const int g = t / nq, st = tile_of(t - (t / nq) * nq), h = hk * G + g;
    tq.load(a.q, b, h, 32 * st, S, D, vec);
    tg.load(a.dout, b, h, 32 * st, S, D, vec);
    if (tid < 32) {
      const int q = 32 * st + tid;
      dnext = q < S ? docb[q] : 0;
    } else if (tid < 96) {  // lse (threads 32..63) and delta (64..95) of the sub-tile's rows
      const int q = 32 * st + (tid & 31);
      const int64_t ri = ((int64_t)b * a.Hq + h) * S + q;
      lnext = q < S ? (tid < 64 ? a.lse[ri] : a.delta[ri]) : 0.f;
    }
  };
  fetch(i0);
  for (int t = i0; t < i1; ++t) {
    __syncthreads();
    tq.store_rs(Qs, vec);
    tq.store_tr(Qt, vec);
    tg.store_rs(Gs, vec);
    tg.store_tr(Gt, vec);
    if (tid < 32) qd[tid] = dnext;
    else if (tid < 64) ls[tid - 32] = lnext;
    else if (tid < 96) dls[tid - 64] = lnext;
    __syncthreads();
    const int q0 = 32 * tile_of(t % nq);
    if (t + 1 < i1) fetch(t + 1);
    unsigned okm = 0;  // bit r: pair (query q0 + crow(hh, r), KV row kv) allowed
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int q = q0 + crow(hh, r);
      okm |= (unsigned)(kvv && q < S && q >= kv && qd[crow(hh, r)] == kvdoc) << r;
    }
    if (__builtin_amdgcn_ballot_w64(okm != 0) == 0) continue;
    f32x16_t sacc = zero16(), pacc = zero16();
#pragma unroll
    for (int q4 = 0; q4 < NS / 4; ++q4)
      if (8 * q4 < D) {
        const f32x4_t qa = rs4<DP>(Qs, l32, hh, q4), ga = rs4<DP>(Gs, l32, hh, q4);
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          sacc = mfma(qa[x], kf[4 * q4 + x], sacc);  // S = Q K^T (lane <-> KV column)
          pacc = mfma(ga[x], vf[4 * q4 + x], pacc);  // dP = dO V^T
        }
      }
    float pv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qr = crow(hh, r);
      const float p = (okm >> r) & 1 ? fast_exp2(sacc[r] - ls[qr]) : 0.f;
      pv[r] = p;
      sacc[r] = p * (pacc[r] - dls[qr]);  // dS
    }
    // dV^T += dO^T P, dK^T += Q^T dS (step r pairs query rows crow(0, r), crow(1, r))
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      if (32 * db < D) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4_t ga = tr4(Gt, db, l32, hh, g), qa = tr4(Qt, db, l32, hh, g);
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            dvacc[db] = mfma(ga[x], pv[4 * g + x], dvacc[db]);
            dkacc[db] = mfma(qa[x], sacc[4 * g + x], dkacc[db]);
          }
        }
      }
  }
  if (!kvv) return;
  const int64_t ro = ((int64_t)bh * S + kv) * D + chunk * a.pstride;
  float *dkr = nch == 1 ? a.dk.row(b, hk, kv) : a.part + ro;
  float *dvr = nch == 1 ? a.dv.row(b, hk, kv) : a.part2 + ro;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 32 * db + crow(hh, r);
      if (d < D) {
        dkr[d] = dkacc[db][r] * a.scale;
        dvr[d] = dvacc[db][r];
      }
    }
}

// dK / dV of KV tiles with more than one chunk: the chunk partials added in
// chunk order (run-to-run deterministic), one thread per output element.
__global__ __launch_bounds__(256) void attn_f32_sum_chunks(Args a) {
  const int heads = a.Hkv;
  const int64_t rows = (int64_t)a.B * heads * a.S;
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= rows * a.D) return;
  const int64_t row = e / a.D;
  const int d = (int)(e - row * a.D);
  const int S = a.S;
  const int q = (int)(row % S), bh = (int)(row / S);
  const int nt = (S + kRows - 1) / kRows;
  const int nch = a.nch[bh * nt + q / kRows];
  if (nch <= 1) return;
  const int b = bh / heads, hh = bh % heads;
  float s0 = 0.f, s1 = 0.f;
  for (int c = 0; c < nch; ++c) {
    s0 += a.part[c * a.pstride + e];
    s1 += a.part2[c * a.pstride + e];
  }
  a.dk.row(b, hh, q)[d] = s0;
  a.dv.row(b, hh, q)[d] = s1;
}

View view_of(const pb_bhsd *t) {
  return View{static_cast<float *>(t->data), t->stride_b, t->stride_h, t->stride_s};
}

bool rows_aligned(const pb_bhsd *t) {
  return reinterpret_cast<uintptr_t>(t->data) % 16 == 0 && t->stride_b % 4 == 0 &&
         t->stride_h % 4 == 0 && t->stride_s % 4 == 0;
}

int check(const char *what, int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t d) {
  PB_CHECK_ARG(b >= 1 && hq >= 1 && hkv >= 1 && s >= 1 && d >= 1,
               "%s: bad shape b=%lld hq=%lld hkv=%lld s=%lld d=%lld", what, (long long)b,
               (long long)hq, (long long)hkv, (long long)s, (long long)d);
  PB_CHECK_ARG(hq % hkv == 0, "%s: query heads (%lld) not a multiple of kv heads (%lld)", what,
               (long long)hq, (long long)hkv);
  PB_CHECK_SUPPORTED(d <= 128, "%s: head_dim %lld > 128 is not supported", what, (long long)d);
  PB_CHECK_SUPPORTED(s < (1LL << 30) && b * hq * ((s + kRows - 1) / kRows) < (1LL << 31) &&
                         b * hq * s < (1LL << 40),
                     "%s: problem too large", what);
  return PB_OK;
}

// Chunks per tile for a grid of `tiles` workgroups: split only small grids,
// aiming at ~2048 workgroups (at most 8 chunks).
inline int splits_for(int64_t tiles) {
  if (tiles >= 1024) return 1;
  const int64_t n = (2048 + tiles - 1) / tiles;
  return (int)(n < 8 ? n : 8);
}

inline int64_t al256(int64_t bytes) { return (bytes + 255) / 256 * 256; }

// Workspace of pb_attn_bwd_f32: delta [B*Hq*S], then (dK/dV grid split)
// nch [KV tiles] int and the dK and dV partials [nsplit][B*Hkv*S][D] each.
struct Layout {
  int nsplit;
  int64_t nch, part_k, part_v, total;
};

inline Layout bwd_layout(int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t d) {
  Layout L = {};
  const int64_t nt = (s + kRows - 1) / kRows, kvrows = b * hkv * s;
  L.nsplit = splits_for(b * hkv * nt);
  int64_t off = al256(b * hq * s * 4);  // delta
  if (L.nsplit > 1) {
    L.nch = off;
    off += al256(b * hkv * nt * 4);
    L.part_k = off;
    off += al256(L.nsplit * kvrows * d * 4);
    L.part_v = off;
    off += al256(L.nsplit * kvrows * d * 4);
  }
  L.total = off;
  return L;
}

}  // namespace attn32
}  // namespace pb

using pb::attn32::Args;

extern "C" int64_t pb_attn_bwd_f32_workspace_bytes(int64_t b, int64_t hq, int64_t hkv, int64_t s,
                                                    int64_t d) {
  if (b < 1 || hq < 1 || hkv < 1 || s < 1 || d < 1) return 0;
  return pb::attn32::bwd_layout(b, hq, hkv, s, d).total;
}

extern "C" int pb_attn_fwd_f32(const pb_bhsd *q, const pb_bhsd *k, const pb_bhsd *v,
                               const pb_bhsd *out, float *lse, const int64_t *doc_ids,
                               int64_t doc_stride, int64_t b, int64_t hq, int64_t hkv, int64_t s,
                               int64_t d, float scale, void *stream) {
  using namespace pb;
  using namespace pb::attn32;
  clear_error();
  int rc = check("pb_attn_fwd_f32", b, hq, hkv, s, d);
  if (rc) return rc;
  PB_CHECK_ARG(q && k && v && out && lse && doc_ids, "pb_attn_fwd_f32: null argument");
  PB_CHECK_ARG(scale > 0.f, "pb_attn_fwd_f32: softmax scale must be positive");
  Args a = {};
  a.q = view_of(q); a.k = view_of(k); a.v = view_of(v); a.o = view_of(out);
  a.lse = lse;
  a.doc = doc_ids; a.doc_sb = doc_stride;
  a.B = (int)b; a.Hq = (int)hq; a.Hkv = (int)hkv; a.S = (int)s; a.D = (int)d;
  a.scale = scale;
  a.vec = d % 4 == 0 && rows_aligned(k) && rows_aligned(v);
  const dim3 grid((unsigned)(b * hq * ((s + kRows - 1) / kRows))), block(64 * kWaves);
  hipStream_t st = as_stream(stream);
  if (d <= 32) hipLaunchKernelGGL(attn_fwd_f32<32>, grid, block, 0, st, a);
  else if (d <= 64) hipLaunchKernelGGL(attn_fwd_f32<64>, grid, block, 0, st, a);
  else hipLaunchKernelGGL(attn_fwd_f32<128>, grid, block, 0, st, a);
  return launch_status("pb_attn_fwd_f32");
}

extern "C" int pb_attn_bwd_f32(const pb_bhsd *q, const pb_bhsd *k, const pb_bhsd *v,
                               const pb_bhsd *out, const pb_bhsd *dout, const pb_bhsd *dq,
                               const pb_bhsd *dk, const pb_bhsd *dv, const float *lse,
                               void *workspace, const int64_t *doc_ids, int64_t doc_stride,
                               int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t d,
                               float scale, void *stream) {
  using namespace pb;
  using namespace pb::attn32;
  clear_error();
  int rc = check("pb_attn_bwd_f32", b, hq, hkv, s, d);
  if (rc) return rc;
  PB_CHECK_ARG(q && k && v && out && dout && dq && dk && dv && lse && workspace && doc_ids,
               "pb_attn_bwd_f32: null argument");
  PB_CHECK_ARG(scale > 0.f, "pb_attn_bwd_f32: softmax scale must be positive");
  const Layout L = bwd_layout(b, hq, hkv, s, d);
  char *ws = static_cast<char *>(workspace);
  Args a = {};
  a.q = view_of(q); a.k = view_of(k); a.v = view_of(v); a.o = view_of(out);
  a.dout = view_of(dout); a.dq = view_of(dq); a.dk = view_of(dk); a.dv = view_of(dv);
  a.lse = const_cast<float *>(lse);
  a.delta = reinterpret_cast<float *>(ws);
  a.doc = doc_ids; a.doc_sb = doc_stride;
  a.B = (int)b; a.Hq = (int)hq; a.Hkv = (int)hkv; a.S = (int)s; a.D = (int)d;
  a.scale = scale;
  a.vec = d % 4 == 0 && rows_aligned(q) && rows_aligned(k) && rows_aligned(v) &&
          rows_aligned(dout);
  hipStream_t st = as_stream(stream);
  const int64_t nt = (s + kRows - 1) / kRows;
  const dim3 block(64 * kWaves);
  // dQ first: it writes delta, which the dK/dV kernel reads.
  const dim3 gq((unsigned)(b * hq * nt));
  if (d <= 32) hipLaunchKernelGGL(attn_bwd_dq_f32<32>, gq, block, 0, st, a);
  else if (d <= 64) hipLaunchKernelGGL(attn_bwd_dq_f32<64>, gq, block, 0, st, a);
  else hipLaunchKernelGGL(attn_bwd_dq_f32<128>, gq, block, 0, st, a);
  rc = launch_status("pb_attn_bwd_f32(dq)");
  if (rc) return rc;
  Args akv = a;
  akv.nsplit = L.nsplit;
  if (akv.nsplit > 1) {
    akv.nch = reinterpret_cast<int *>(ws + L.nch);
    akv.part = reinterpret_cast<float *>(ws + L.part_k);
    akv.part2 = reinterpret_cast<float *>(ws + L.part_v);
    akv.pstride = b * hkv * s * d;
  }
  const dim3 gkv((unsigned)(b * hkv * nt * akv.nsplit));
  if (d <= 32) hipLaunchKernelGGL(attn_bwd_dkdv_f32<32>, gkv, block, 0, st, akv);
  else if (d <= 64) hipLaunchKernelGGL(attn_bwd_dkdv_f32<64>, gkv, block, 0, st, akv);
  else hipLaunchKernelGGL(attn_bwd_dkdv_f32<128>, gkv, block, 0, st, akv);
  rc = launch_status("pb_attn_bwd_f32(dkdv)");
  if (rc || akv.nsplit == 1) return rc;
  hipLaunchKernelGGL(attn_f32_sum_chunks, dim3((unsigned)((b * hkv * s * d + 255) / 256)), dim3(256),
                     0, st, akv);
  return launch_status("pb_attn_bwd_f32(dkdv sum)");
}
