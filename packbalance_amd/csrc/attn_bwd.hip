// Document-masked GQA attention backward for gfx950 (bf16 in, fp32 accumulate).
//
// Reference: the FlexAttention backward of packbalance/model/attention.py:116-122
// (gradients of softmax(scale * Q K^T | doc mask) V, dK/dV summed over each
// GQA group as enable_gqa does).  With P = softmax, D_i = rowsum(dO_i * O_i):
//   dV = P^T dO,  dP = dO V^T,  dS = P * (dP - D),
//   dQ = scale * dS K,  dK = scale * dS^T Q.
//
// Kept dS (head dim 128 on a full grid, AttnConfig::ds): attn_bwd_delta forms
// D, attn_bwd_dkdv_pairs<128, true> also stores its bf16 dS tiles, and
// attn_bwd_dq_ds forms dQ = scale * dS K from them; otherwise two kernels.
// No atomics on either path (results are run-to-run deterministic):
//   attn_bwd_dq     one workgroup per (pack, query head, 128-row query tile),
//                   shaped like the forward: lane <-> query row.  It first forms
//                   D = rowsum(dO * O) from its register-resident rows (stored
//                   for the second kernel), then recomputes S^T and dP^T per
//                   64-row KV tile and accumulates dQ^T = K^T dS^T, reading K^T
//                   fragments from the row-major K tile with ds_read_b64_tr_b16.
//   attn_bwd_dkdv   one workgroup per (pack, KV head, KV tile of 32*W rows);
//                   wave w owns 32 KV rows with K and V fragments in
//                   registers.  It walks every query head of its GQA group and
//                   every 64-row query tile the plan lists for the KV tile, so
//                   dK/dV accumulate in registers across the whole group.  When
//                   the grid would be too small to fill the GPU (AttnConfig
//                   split), each query head gets its own workgroup and writes
//                   fp32 partials that attn_bwd_reduce sums over the group.  S = Q K^T
//                   is computed with lane <-> KV row, so P^T and dS^T feed the
//                   dV / dK MFMAs straight from the accumulators; the Q^T / dO^T
//                   operands are read from the row-major LDS tiles with
//                   ds_read_b64_tr_b16, and the next tile is prefetched into
//                   registers while the current one is computed.
#include <algorithm>
#include <type_traits>

#include "attn_common.hpp"

namespace pb {
namespace attn {


struct View {
  bf16_t *p;
  int64_t sb, sh, ss;
  __device__ __forceinline__ bf16_t *row(int b, int h, int64_t s) const {
    return p + b * sb + h * sh + s * ss;
  }
};

struct BwdArgs {
  View q, k, v, o, dout, dq, dk, dv;
  const float *lse;
  float *delta;
  const int64_t *doc;
  int64_t doc_sb;
  const int32_t *qcnt, *qlist;  // dQ plan (by query tile)
  const int32_t *kcnt, *klist;  // dK/dV plan (by KV tile)
  float *dk_part, *dv_part;     // split: fp32 [B][Hq][S][D] partials
  // split, pipelined kernel: a KV tile whose list has at least kv_chunk steps
  // is walked by two workgroups (first and second half of its steps); the
  // second writes its partials here.  0: whole lists, these are unused.
  float *dk_part2, *dv_part2;
  int kv_chunk, kv_tile;
  // dQ KV split: KV tiles per workgroup (0: whole list), unscaled fp32 dQ
  // partials [split][B][Hq][S][D] of query tiles with more than one chunk.
  int dq_chunk;
  float *dq_part;
  // Kept dS blocks (AttnConfig::ds): the region of pack b, KV head hk starts
  // at ds + (b * Hkv + hk) * ds_pair bytes.
  char *ds;
  int64_t ds_pair;
  int B, Hq, Hkv, S, D;
  int nqt_dq, nkt_dq, nqt_kv, nkt_kv;
  float sl2, scale;
  int vec;
};

// Split dK/dV on the pipelined kernel: KV tiles whose step list is at least
// this long are walked by two workgroups (a 2048-token document's first KV
// tiles have 64 steps per head where the mean over a cfg2 pack is ~20, and
// the longest list sets the launch time).
constexpr int kKvChunkSteps = 16;

// ---------------------------------------------------------------- dK, dV
template <int DP, int WAVES, bool SPLIT>
__global__ __launch_bounds__(64 * WAVES) void attn_bwd_dkdv(BwdArgs a) {
  constexpr int NT = 64 * WAVES;
  constexpr int BN = 32 * WAVES, BM = kQStep;
  constexpr int QP = DP + 8;  // row-major pitch (elements)
  constexpr int NDK = DP / 16, NDB = DP / 32, CH = DP / 8;
  constexpr int NCH = BM * CH;             // 16-byte chunks of one [BM x DP] tile
  constexpr int NLD = (2 * NCH + NT - 1) / NT;  // chunks per thread (Q and dO)
  __shared__ __align__(16) bf16_t Qs[BM * QP];
  __shared__ __align__(16) bf16_t Gs[BM * QP];  // dO
  __shared__ float lse_s[BM], dlt_s[BM];
  __shared__ int64_t qdoc_s[BM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hh = lane >> 5, l32 = lane & 31;
  // Grid: (KV tile, pack, KV head[, group member]); early KV tiles are
  // attended by the most query tiles, so they come first.
  const int Gfull = a.Hq / a.Hkv;
  const int G = SPLIT ? 1 : Gfull;
  const int per_tile = a.B * a.Hkv * (SPLIT ? Gfull : 1);
  const int kt = (int)(blockIdx.x / per_tile);
  int rem = (int)(blockIdx.x % per_tile);
  const int g0 = SPLIT ? rem % Gfull : 0;
  if (SPLIT) rem /= Gfull;
  const int b = rem / a.Hkv, hk = rem - (rem / a.Hkv) * a.Hkv;
  const bool vec = a.vec != 0;
  const int64_t *docb = a.doc + b * a.doc_sb;

  const int kv = kt * BN + wave * 32 + l32;
  const bool kvvalid = kv < a.S;
  const int64_t kvdoc = kvvalid ? docb[kv] : 0;
  bf16x8_t kf[NDK], vf[NDK];
  {
    const int64_t r = kvvalid ? kv : 0;
    const bf16_t *krow = a.k.row(b, hk, r), *vrow = a.v.row(b, hk, r);
#pragma unroll
    for (int dk = 0; dk < NDK; ++dk) {
      kf[dk] = load_row8(krow, 16 * dk + 8 * hh, a.D, kvvalid, vec);
      vf[dk] = load_row8(vrow, 16 * dk + 8 * hh, a.D, kvvalid, vec);
    }
  }
  f32x16_t dk_acc[NDB], dv_acc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) {
    dk_acc[i] = zero16();
    dv_acc[i] = zero16();
  }

  const int cnt = a.kcnt[b * a.nkt_kv + kt];
  const int32_t *lst = a.klist + ((int64_t)b * a.nkt_kv + kt) * a.nqt_kv;
  const int steps = cnt * G;  // (query head of the group, query tile) pairs

  // Register prefetch of one step's Q / dO tiles and per-row scalars.
  bf16x8_t pre[NLD];
  float pre_lse = 0.f, pre_dlt = 0.f;
  int64_t pre_doc = 0;
  auto fetch = [&](int step) {
    const int g = step / cnt, it = step - (step / cnt) * cnt;
    const int h = hk * Gfull + g0 + g;
    const int q0 = plan_tile(lst[it]) * BM;
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int c = tid + NT * i;
      if (c < 2 * NCH) {
        const int which = c / NCH, cc = c - which * NCH;
        const int row = cc / CH, col = (cc % CH) * 8;
        const int qr = q0 + row;
        const bool ok = qr < a.S;
        const View &src = which ? a.dout : a.q;
        pre[i] = load_row8(src.row(b, h, ok ? qr : 0), col, a.D, ok, vec);
      }
    }
    for (int r = tid; r < BM; r += NT) {  // NT >= BM: one row per thread
      const int qr = q0 + r;
      const bool ok = qr < a.S;
      const int64_t o = ((int64_t)b * a.Hq + h) * a.S + (ok ? qr : 0);
      pre_lse = ok ? a.lse[o] : 0.f;
      pre_dlt = ok ? a.delta[o] : 0.f;
      pre_doc = ok ? docb[qr] : 0;
    }
  };

  if (steps > 0) fetch(0);
  for (int step = 0; step < steps; ++step) {
    const int it = step % cnt;
    const int e = lst[it];
    const int q0 = plan_tile(e) * BM;
    const bool full = plan_full(e);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int c = tid + NT * i;
      if (c < 2 * NCH) {
        const int which = c / NCH, cc = c - which * NCH;
        const int row = cc / CH, col = (cc % CH) * 8;
        *reinterpret_cast<bf16x8_t *>(&(which ? Gs : Qs)[row * QP + col]) = pre[i];
      }
    }
    if (tid < BM) {
      lse_s[tid] = pre_lse;
      dlt_s[tid] = pre_dlt;
      qdoc_s[tid] = pre_doc;
    }
    __syncthreads();
    if (step + 1 < steps) fetch(step + 1);

    // S = Q K^T, dP = dO V^T: two 32-query blocks x this wave's 32 KV rows.
    bf16x8_t pf[4], dsf[4];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      f32x16_t sacc = zero16(), pacc = zero16();
#pragma unroll
      for (int dk = 0; dk < NDK; ++dk) {
        const int off = (32 * qb + l32) * QP + 16 * dk + 8 * hh;
        sacc = mfma32(*reinterpret_cast<const bf16x8_t *>(&Qs[off]), kf[dk], sacc);
        pacc = mfma32(*reinterpret_cast<const bf16x8_t *>(&Gs[off]), vf[dk], pacc);
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int qr = 32 * qb + 8 * (j >> 2) + 4 * hh + (j & 3);
        const int q = q0 + qr;
        const bool ok = full || (q < a.S && kvvalid && q >= kv && qdoc_s[qr] == kvdoc);
        const float p = ok ? fast_exp2(fmaf(sacc[j], a.sl2, -lse_s[qr])) : 0.f;
        pf[2 * qb + (j >> 3)][j & 7] = (bf16_t)p;
        dsf[2 * qb + (j >> 3)][j & 7] = (bf16_t)(p * (pacc[j] - dlt_s[qr]));
      }
    }
    // dV += P^T dO, dK += dS^T Q; B operands = column fragments of the tiles.
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int qk = 0; qk < 4; ++qk) {
        dv_acc[db] = mfma32(pf[qk], lds_col_frag(Gs, QP, 16 * qk, 32 * db, lane), dv_acc[db]);
        dk_acc[db] = mfma32(dsf[qk], lds_col_frag(Qs, QP, 16 * qk, 32 * db, lane), dk_acc[db]);
      }
  }
  // Accumulators: lane <-> head-dim column, register j <-> KV row of the wave.
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    const int d = 32 * db + l32;
    if (d >= a.D) continue;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int kvr = kt * BN + wave * 32 + 8 * (j >> 2) + 4 * hh + (j & 3);
      if (kvr < a.S) {
        if constexpr (SPLIT) {
          const int64_t o = (((int64_t)b * a.Hq + hk * Gfull + g0) * a.S + kvr) * a.D + d;
          a.dk_part[o] = dk_acc[db][j];
          a.dv_part[o] = dv_acc[db][j];
        } else {
          a.dk.row(b, hk, kvr)[d] = (bf16_t)(dk_acc[db][j] * a.scale);
          a.dv.row(b, hk, kvr)[d] = (bf16_t)dv_acc[db][j];
        }
      }
    }
  }
}

// ---------------------------------------------------------------- dK, dV (pipelined)
// Grid decode of the KV-major kernel for L2 reuse: workgroup i runs on XCD
// i % 8; each XCD takes whole (pack, KV head[, member]) pairs and walks their
// KV tiles in order, so the workgroups resident on one XCD stream the same
// Q / dO rows through its L2 (each KV tile reads every query tile at or after
// it).  Identity map when the pair count is not a multiple of 8.
__device__ __forceinline__ void decode_kv_major(int bid, int nkt, int npairs, int &kt, int &pair) {
  if (npairs % 8 == 0) {
    const int x = bid & 7, j = bid >> 3;
    pair = (j / nkt) * 8 + x;
    kt = j - (j / nkt) * nkt;
  } else {
    pair = bid / nkt;
    kt = bid - pair * nkt;
  }
}

// One step of the pipelined dK/dV walk: query head, first query row, plan
// entry.  (Declared at namespace scope: a struct local to the kernel template
// keeps clang from emitting the kernel's host stub.)
struct DkdvStep {
  int h, q0, e;
};

// Pipelined dK/dV (16-byte aligned views and documents, D == DP in {64, 128},
// sequence a multiple of 64).  Wave w owns 32 KV rows with K and V fragments
// in registers and dK/dV accumulators.  The workgroup walks steps t = (query
// sub-tile of 32 rows, query head of the group), sub-tile outer: per step
// S = Q K^T and dP = dO V^T (lane <-> KV row), P = exp2(S*scale*log2e -
// lse), dS = P*(dP - delta), then dV += P^T dO and dK += dS^T Q with the Q /
// dO column fragments read by ds_read_b64_tr_b16 from the same swizzled LDS
// tiles the row fragments come from.  Q, dO, lse/delta and the query
// documents arrive by DMA through a 4-slot ring (steps t+1 .. t+3 in flight
// while t is computed, one barrier per step); the MFMAs of S(t+1) and
// dP(t+1) are interleaved with the P/dS math of step t.
// Q / dO row-fragment reads in flight ahead of their MFMAs: two at head dim
// 64 (the registers this frees fit two waves per SIMD), all of them at 128
// (one wave per SIMD either way; streaming them measured slower there).
template <int DP>
constexpr int kAheadDkdv = DP == 64 ? 2 : DP / 16;

// Head dim 64 fits two waves per SIMD (with the row fragments streamed);
// head dim 128 needs ~400 registers and runs one.
template <int DP, int WAVES, bool SPLIT>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(DP == 64 ? 2 : 1, DP == 64 ? 2 : 1)))
void attn_bwd_dkdv_pipe(BwdArgs a) {
  constexpr int NT = 64 * WAVES, BN = 32 * WAVES;
  constexpr int NDK = DP / 16, NDB = DP / 32;
  constexpr int HB = 32 * DP * 2;  // bytes of one 32-row sub-tile
  using Dma = TileDma<DP, 32, NT>;
  constexpr int NDMA = Dma::NDMA;
  constexpr int NVF = 2 * NDB;  // column fragments of one operand per step
  // Ring slots are separate LDS objects (see attn_fwd_pipe).
  __shared__ __align__(16) char qs0[HB], qs1[HB], qs2[HB], qs3[HB];
  __shared__ __align__(16) char gs0[HB], gs1[HB], gs2[HB], gs3[HB];
  __shared__ __align__(16) float ld0[64], ld1[64], ld2[64], ld3[64];  // lse[32], delta[32]
  __shared__ __align__(16) int64_t qd0[32], qd1[32], qd2[32], qd3[32];
  auto qslot = [&](auto Rc) -> char * {
    constexpr int R = decltype(Rc)::value;
    if constexpr (R == 0) return qs0; else if constexpr (R == 1) return qs1;
    else if constexpr (R == 2) return qs2; else return qs3;
  };
  auto gslot = [&](auto Rc) -> char * {
    constexpr int R = decltype(Rc)::value;
    if constexpr (R == 0) return gs0; else if constexpr (R == 1) return gs1;
    else if constexpr (R == 2) return gs2; else return gs3;
  };
  auto lslot = [&](auto Rc) -> float * {
    constexpr int R = decltype(Rc)::value;
    if constexpr (R == 0) return ld0; else if constexpr (R == 1) return ld1;
    else if constexpr (R == 2) return ld2; else return ld3;
  };
  auto dslot = [&](auto Rc) -> int64_t * {
    constexpr int R = decltype(Rc)::value;
    if constexpr (R == 0) return qd0; else if constexpr (R == 1) return qd1;
    else if constexpr (R == 2) return qd2; else return qd3;
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hh = lane >> 5, l32 = lane & 31;
  const int Gfull = a.Hq / a.Hkv;
  const int G = SPLIT ? 1 : Gfull;
  int kt, pair, bid = (int)blockIdx.x, chunk = 0;
  if (SPLIT && a.kv_chunk > 0) {  // grid = two copies: chunk 0, then chunk 1
    const int nb = a.nkt_kv * a.B * a.Hkv * Gfull;
    chunk = bid / nb;
    bid -= chunk * nb;
  }
  decode_kv_major(bid, a.nkt_kv, a.B * a.Hkv * (SPLIT ? Gfull : 1), kt, pair);
  const int g0 = SPLIT ? pair % Gfull : 0;
  const int bh = SPLIT ? pair / Gfull : pair;
  const int b = bh / a.Hkv, hk = bh - (bh / a.Hkv) * a.Hkv;
  const int S = a.S;
  const int64_t *docb = a.doc + b * a.doc_sb;
  const float sl2 = a.sl2;

  const int kv = kt * BN + wave * 32 + l32;
  const bool kvvalid = kv < S;
  const int kvr = kvvalid ? kv : S - 1;
  const int64_t kvdoc = docb[kvr];
  bf16x8_t kf[NDK], vf[NDK];
  {
    const bf16_t *krow = a.k.row(b, hk, kvr), *vrow = a.v.row(b, hk, kvr);
#pragma unroll
    for (int dk = 0; dk < NDK; ++dk) {
      kf[dk] = *reinterpret_cast<const bf16x8_t *>(krow + 16 * dk + 8 * hh);
      vf[dk] = *reinterpret_cast<const bf16x8_t *>(vrow + 16 * dk + 8 * hh);
    }
  }
  f32x16_t dk_acc[NDB], dv_acc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) {
    dk_acc[i] = zero16();
    dv_acc[i] = zero16();
  }

  uint32_t qoff[NDMA], goff[NDMA];
  Dma::offsets(a.q.ss, wave, lane, qoff);
  Dma::offsets(a.dout.ss, wave, lane, goff);
  // Per-lane fragment offsets within a sub-tile (see attn_fwd_pipe).
  int roffs[NDK], coffs[NDB][2];
  {
    const int j = lane & 15, g = lane >> 4;
#pragma unroll
    for (int dk = 0; dk < NDK; ++dk) {
      roffs[dk] = SwzTile<DP>::off(l32, 16 * dk + 8 * hh);
      asm volatile("" : "+v"(roffs[dk]));
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int col = 32 * db + 16 * (g & 1) + 4 * (j & 3);
      const int row = 4 * hh + (j >> 2);
      coffs[db][0] = SwzTile<DP>::off(row, col);
      coffs[db][1] = SwzTile<DP>::off(row + 8, col);
      asm volatile("" : "+v"(coffs[db][0]), "+v"(coffs[db][1]));
    }
  }
  auto rfrag = [&](const char *t, int dk) {
    return *reinterpret_cast<const bf16x8_t *>(t + roffs[dk]);
  };
  auto cfrag = [&](const char *t, int f) {  // f = qk * NDB + db
    const char *base = t + (f / NDB) * 16 * DP * 2;
    const int db = f % NDB;
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base + coffs[db][0]));
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base + coffs[db][1]));
    typedef short i16x8_t __attribute__((ext_vector_type(8)));
    i16x8_t r = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return *reinterpret_cast<bf16x8_t *>(&r);
  };

  const int cnt = a.kcnt[b * a.nkt_kv + kt];
  const int U = 2 * cnt;  // 32-row query sub-tiles
  int T = G * U;          // steps: sub-tile outer, head of the group inner
  int t0 = 0;             // first step of this workgroup's share
  if (SPLIT && a.kv_chunk > 0) {
    if (T >= a.kv_chunk) {  // halves: chunk 0 takes [0, T/2), chunk 1 the rest
      const int h = T / 2;
      t0 = chunk ? h : 0;
      T = chunk ? T - h : h;
    } else if (chunk) {
      return;  // short list: chunk 0 walks it whole (uniform over the workgroup)
    }
  }
  const int32_t *lst = a.klist + ((int64_t)b * a.nkt_kv + kt) * a.nqt_kv;
  // Step t -> (query head, first query row, plan entry); steps past the last
  // repeat it (their DMA lands in slots nobody reads any more).
  auto step_of = [&](int t, int e) {
    const int tc = (t < T ? t : T - 1) + t0;
    const int u = tc / G, g = tc - (tc / G) * G;
    DkdvStep s;
    s.h = hk * Gfull + g0 + g;
    s.e = e;
    s.q0 = plan_tile(e) * kQStep + 32 * (u & 1);
    return s;
  };
  auto entry = [&](int t) {
    const int tc = (t < T ? t : T - 1) + t0;
    return lst[(tc / G) >> 1];
  };

  // DMA of one step: lse/delta (wave 0) and query documents (wave 1 % W)
  // first, then the Q and dO sub-tiles.
  // One buffer resource for each of Q and dO over the rows of this
  // workgroup's query heads (h0 .. h0 + G - 1); a step's DMA passes its byte
  // offset as the scalar offset (the host keeps these extents below 2 GiB on
  // this path).
  const int h0 = hk * Gfull + g0;
  const auto qrs = buf_rsrc(a.q.row(b, h0, 0), 0x7fffffff);
  const auto grs = buf_rsrc(a.dout.row(b, h0, 0), 0x7fffffff);
  const uint32_t qsh2 = (uint32_t)(a.q.sh * 2), qss2 = (uint32_t)(a.q.ss * 2);
  const uint32_t gsh2 = (uint32_t)(a.dout.sh * 2), gss2 = (uint32_t)(a.dout.ss * 2);
  auto dma_step = [&](const DkdvStep &s, auto Rc) {
    const int64_t ro = ((int64_t)b * a.Hq + s.h) * S + s.q0;
    // lse to LDS floats [0, 32) (lanes 0-7), delta to [32, 64) (lanes 8-15):
    // two DMAs, since a buffer resource is wave-uniform.
    if (wave == 0 && lane < 8) dma16(a.lse + ro, 0x7fffffff, 16 * lane, lslot(Rc));
    if (wave == 0 && lane >= 8 && lane < 16) dma16(a.delta + ro, 0x7fffffff, 16 * (lane - 8), lslot(Rc));
    if (wave == (WAVES > 1 ? 1 : 0) && lane < 16)
      dma16(docb + s.q0, 0x7fffffff, 16 * lane, dslot(Rc));
    const uint32_t dh = (uint32_t)(s.h - h0), q0 = (uint32_t)s.q0;
    Dma::copy_rs(qrs, dh * qsh2 + q0 * qss2, qoff, qslot(Rc), wave);
    Dma::copy_rs(grs, dh * gsh2 + q0 * gss2, goff, gslot(Rc), wave);
  };

  // Element mask of a PARTIAL step: same document, kv <= q (q < S always).
  // Tests as bitwise ands (no per-element branch), with two wave-uniform
  // shortcuts: a step wholly at or after the wave's last KV row needs no
  // causal test, a CAUSAL plan tile no document test.  KV rows past the
  // sequence end are left unmasked: their dK / dV are never stored.
  // kv <= q0 + pi_row(hh, j)  <=>  kv - q0 - 4hh <= 8(j/4) + j%4.
  const int kvmax = kt * BN + wave * 32 + 31;
  auto mask = [&](f32x16_t &sv, int e, int q0, const int64_t *qd) {
    const bool diag = q0 < kvmax;
    const int rel = kv - q0 - 4 * hh;
    if (plan_causal(e)) {
      if (!diag) return;
#pragma unroll
      for (int j = 0; j < 16; ++j) sv[j] = rel <= 8 * (j >> 2) + (j & 3) ? sv[j] : -INFINITY;
      return;
    }
    int64_t dq[16];
    lds_docs16(qd, hh, dq);
    if (diag) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const bool ok = (rel <= 8 * (j >> 2) + (j & 3)) & (dq[j] == kvdoc);
        sv[j] = ok ? sv[j] : -INFINITY;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) sv[j] = dq[j] == kvdoc ? sv[j] : -INFINITY;
    }
  };

  // P and dS of one step for elements j, j+1 (query rows 8(j/4) + 4hh + j%4).
  // The packed results pass through an empty volatile asm so they are formed
  // where this call sits in the MFMA schedule, not sunk towards their use.
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  auto pds2 = [&](int j, const f32x16_t &sc, const f32x16_t &pc, const float (&lse)[16],
                  const float (&dlt)[16], bf16x8_t (&pf)[2], bf16x8_t (&dsf)[2]) {
    bf16x2_t pp, dd;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float p = fast_exp2(fmaf(sc[j + i], sl2, -lse[j + i]));
      pp[i] = (bf16_t)p;
      dd[i] = (bf16_t)(p * (pc[j + i] - dlt[j + i]));
    }
    asm volatile("" ::"v"(*reinterpret_cast<uint32_t *>(&pp)), "v"(*reinterpret_cast<uint32_t *>(&dd)));
    pf[j >> 3][j & 7] = pp[0];
    pf[j >> 3][(j & 7) + 1] = pp[1];
    dsf[j >> 3][j & 7] = dd[0];
    dsf[j >> 3][(j & 7) + 1] = dd[1];
  };
  auto load_ld = [&](const float *ld, float (&lse)[16], float (&dlt)[16]) {
#pragma unroll
    for (int jg = 0; jg < 4; ++jg) {
      const float4 l4 = *reinterpret_cast<const float4 *>(ld + 8 * jg + 4 * hh);
      const float4 d4 = *reinterpret_cast<const float4 *>(ld + 32 + 8 * jg + 4 * hh);
      lse[4 * jg] = l4.x; lse[4 * jg + 1] = l4.y; lse[4 * jg + 2] = l4.z; lse[4 * jg + 3] = l4.w;
      dlt[4 * jg] = d4.x; dlt[4 * jg + 1] = d4.y; dlt[4 * jg + 2] = d4.z; dlt[4 * jg + 3] = d4.w;
    }
  };
  auto dvdk = [&](int f, const bf16x8_t &gcol, const bf16x8_t &qcol, const bf16x8_t (&pf)[2],
                  const bf16x8_t (&dsf)[2]) {
    dv_acc[f % NDB] = mfma32(pf[f / NDB], gcol, dv_acc[f % NDB]);
    dk_acc[f % NDB] = mfma32(dsf[f / NDB], qcol, dk_acc[f % NDB]);
  };

  if (T > 0) {
    // Plan entries of steps t+1 .. t+4 for body t (loaded one body ahead).
    int ew[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ew[i] = entry(i + 1);
    const int e0 = entry(0);
    dma_step(step_of(0, e0), I0());
    dma_step(step_of(1, ew[0]), I1());
    dma_step(step_of(2, ew[1]), I2());
    wait_vmcnt<0>();
    __syncthreads();
    f32x16_t sc = zero16(), pc = zero16();
#pragma unroll
    for (int dk = 0; dk < NDK; ++dk) {
      sc = mfma32(rfrag(qs0, dk), kf[dk], sc);
      pc = mfma32(rfrag(gs0, dk), vf[dk], pc);
    }
    if (!plan_full(e0)) mask(sc, e0, step_of(0, e0).q0, qd0);

    auto body = [&](auto Rc, int t) {
      constexpr int R = decltype(Rc)::value;
      using IR = std::integral_constant<int, R>;
      using IR1 = std::integral_constant<int, (R + 1) % 4>;
      using IR3 = std::integral_constant<int, (R + 3) % 4>;
      const int e1 = __builtin_amdgcn_readfirstlane(ew[0]);
      const int e3 = __builtin_amdgcn_readfirstlane(ew[2]);
      const int e4 = entry(t + 5);  // for body t + 1, issued before this body's DMA
      __builtin_amdgcn_sched_barrier(0);
      dma_step(step_of(t + 3, e3), IR3());
      // Step t's lse/delta; step t+1's Q / dO row fragments stream
      // kAheadDkdv steps ahead of their MFMAs.
      float lse[16], dlt[16];
      load_ld(lslot(IR()), lse, dlt);
      bf16x8_t qa[NDK], ga[NDK];
#pragma unroll
      for (int dk = 0; dk < kAheadDkdv<DP>; ++dk) {
        qa[dk] = rfrag(qslot(IR1()), dk);
        ga[dk] = rfrag(gslot(IR1()), dk);
      }
      f32x16_t sn = zero16(), pn = zero16();
      bf16x8_t pf[2], dsf[2];
      __builtin_amdgcn_sched_barrier(0);
      // S(t+1), dP(t+1) MFMAs with the P/dS math of step t between them; the
      // dO / Q column fragments of step t (transposing reads) are spread
      // over the same loop so they have landed when dV / dK need them.
      constexpr int JPS = 16 / NDK;  // elements per head-dim step (2 or 4)
      constexpr int FPS = (NVF + NDK - 1) / NDK;  // column fragments per head-dim step
      bf16x8_t gcol[NVF], qcol[NVF];
#pragma unroll
      for (int dk = 0; dk < NDK; ++dk) {
        if (dk + kAheadDkdv<DP> < NDK) {
          qa[dk + kAheadDkdv<DP>] = rfrag(qslot(IR1()), dk + kAheadDkdv<DP>);
          ga[dk + kAheadDkdv<DP>] = rfrag(gslot(IR1()), dk + kAheadDkdv<DP>);
        }
        sn = mfma32(qa[dk], kf[dk], sn);
        pn = mfma32(ga[dk], vf[dk], pn);
#pragma unroll
        for (int j = dk * JPS; j < (dk + 1) * JPS; j += 2) pds2(j, sc, pc, lse, dlt, pf, dsf);
#pragma unroll
        for (int f = dk * FPS; f < (dk + 1) * FPS && f < NVF; ++f) {
          gcol[f] = cfrag(gslot(IR()), f);
          qcol[f] = cfrag(qslot(IR()), f);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // dV(t) += P^T dO(t), dK(t) += dS^T Q(t); S(t+1) moves into sc alongside.
#pragma unroll
      for (int f = 0; f < NVF; ++f) dvdk(f, gcol[f], qcol[f], pf, dsf);
      sc = sn;
      pc = pn;
      if (!plan_full(e1)) mask(sc, e1, step_of(t + 1, e1).q0, dslot(IR1()));
      wait_vmcnt<2 * NDMA>();
      block_sync_nofence();
      ew[0] = ew[1];
      ew[1] = ew[2];
      ew[2] = ew[3];
      ew[3] = e4;
    };
    int t = 0;
    for (; t + 4 < T; t += 4) {
      body(I0(), t);
      body(I1(), t + 1);
      body(I2(), t + 2);
      body(I3(), t + 3);
    }
    if (t + 1 < T) { body(I0(), t); ++t; }
    if (t + 1 < T) { body(I1(), t); ++t; }
    if (t + 1 < T) { body(I2(), t); ++t; }
    wait_vmcnt<0>();
    // Last step: no S(t+1).
    const int rl = t & 3;
    const char *qt = rl == 0 ? qs0 : rl == 1 ? qs1 : rl == 2 ? qs2 : qs3;
    const char *gt = rl == 0 ? gs0 : rl == 1 ? gs1 : rl == 2 ? gs2 : gs3;
    const float *lt = rl == 0 ? ld0 : rl == 1 ? ld1 : rl == 2 ? ld2 : ld3;
    float lse[16], dlt[16];
    load_ld(lt, lse, dlt);
    bf16x8_t pf[2], dsf[2];
#pragma unroll
    for (int j = 0; j < 16; j += 2) pds2(j, sc, pc, lse, dlt, pf, dsf);
#pragma unroll
    for (int f = 0; f < NVF; ++f) dvdk(f, cfrag(gt, f), cfrag(qt, f), pf, dsf);
  }

  // Accumulators: lane <-> head-dim column, register j <-> KV row of the wave.
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    const int d = 32 * db + l32;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int kvw = kt * BN + wave * 32 + 8 * (j >> 2) + 4 * hh + (j & 3);
      if (kvw < S) {
        if constexpr (SPLIT) {
          const int64_t o = (((int64_t)b * a.Hq + hk * Gfull + g0) * S + kvw) * a.D + d;
          (chunk ? a.dk_part2 : a.dk_part)[o] = dk_acc[db][j];
          (chunk ? a.dv_part2 : a.dv_part)[o] = dv_acc[db][j];
        } else {
          a.dk.row(b, hk, kvw)[d] = (bf16_t)(dk_acc[db][j] * a.scale);
          a.dv.row(b, hk, kvw)[d] = (bf16_t)dv_acc[db][j];
        }
      }
    }
  }
}

// ---------------------------------------------------------------- dK, dV (wave pairs)
// attn_bwd_dkdv_pairs: dK/dV at head dim 128 with the work of each 32-row KV
// block split over a PAIR of waves, so each wave fits 256 registers (the
// one-wave kernel above needs ~400 and runs one wave per SIMD with nothing to
// hide its LDS and dependency latencies).  Same MFMA work, no recomputation:
//   P-wave  (waves 0-1): S(t) = Q(t) K^T, mask, P(t) = exp2(S sl2 - lse),
//                        dV += P(t)^T dO(t); P(t) goes to LDS as the bf16
//                        dV operand it already is.
//   dP-wave (waves 2-3): dP(t) = dO(t) V^T; one step later, when P(t) is
//                        visible, dS(t) = P(t) (dP(t) - delta(t)) and
//                        dK += dS(t)^T Q(t).
// Waves w and w + 2 own the same KV rows and the same lane <-> KV row /
// register <-> query row layout, so P crosses LDS as it sits in registers
// (two 16-byte chunks per lane, conflict-free).  Two pairs make a 64-row KV
// tile and a 4-wave workgroup in under 80 KiB of LDS, so TWO workgroups share
// each CU and one's barrier stalls are covered by the other's work (measured
// against one 8-wave workgroup of four pairs per CU: 2.95 vs 3.3 ms at cfg3).
// LDS: a 4-slot ring (DMA two steps ahead; the dP-wave reads step t-1's Q
// tile), the bf16 P buffers and a step table the prologue fills (first query
// row, head within the group, plan kind per step; query sub-tile outer, head
// inner), so a step's DMA addresses are a table read and two multiplies.  The
// query sub-tiles are walked from the last one down: the workgroups resident
// on one XCD (consecutive KV tiles of one pack and KV head) then read the same
// Q / dO tiles at about the same time, from that XCD's L2 (cfg3 backward
// 4.94 -> 4.82 ms against walking up from each KV tile's diagonal).
// Every step's 32 query rows lie inside the sequence: no buffer bound.  At
// most kPairsMaxSteps steps per KV tile (G * S / 32); longer problems take the
// 2-wave kernel above.
constexpr int kPairsMaxSteps = 1024;

template <int DP, bool DS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_bwd_dkdv_pairs(BwdArgs a) {
  constexpr int NT = 256, NB = 2, BN = 32 * NB;
  constexpr int NDK = DP / 16, NDB = DP / 32;
  constexpr int HB = 32 * DP * 2;  // bytes of one 32-row sub-tile
  constexpr int NVF = 2 * NDB;     // column fragments of one operand per step
  constexpr int NCH = HB / (16 * NT);  // 16-byte DMA chunks per thread and operand
  constexpr int64_t kNoBound = 0x7fffffff;
  static_assert(DP == 128 && NCH == 2, "head dim 128");
  __shared__ __align__(16) char qs0[HB], qs1[HB], qs2[HB], qs3[HB];
  __shared__ __align__(16) char gs0[HB], gs1[HB], gs2[HB], gs3[HB];
  __shared__ __align__(16) float ld0[64], ld1[64], ld2[64], ld3[64];  // lse, delta
  __shared__ __align__(16) int64_t qd0[32], qd1[32], qd2[32], qd3[32];
  // bf16 P(t) of KV block blk as the dV operand: pbuf[t & 1][blk][half][lane] (16 bytes).
  __shared__ __align__(16) u32x4 pbuf[2][NB][2][64];
  __shared__ int32_t steps[kPairsMaxSteps];
  auto qslot = [&](auto Rc) -> char * {
    constexpr int R = decltype(Rc)::value % 4;
    if constexpr (R == 0) return qs0; else if constexpr (R == 1) return qs1;
    else if constexpr (R == 2) return qs2; else return qs3;
  };
  auto gslot = [&](auto Rc) -> char * {
    constexpr int R = decltype(Rc)::value % 4;
    if constexpr (R == 0) return gs0; else if constexpr (R == 1) return gs1;
    else if constexpr (R == 2) return gs2; else return gs3;
  };
  auto lslot = [&](auto Rc) -> float * {
    constexpr int R = decltype(Rc)::value % 4;
    if constexpr (R == 0) return ld0; else if constexpr (R == 1) return ld1;
    else if constexpr (R == 2) return ld2; else return ld3;
  };
  auto dslot = [&](auto Rc) -> int64_t * {
    constexpr int R = decltype(Rc)::value % 4;
    if constexpr (R == 0) return qd0; else if constexpr (R == 1) return qd1;
    else if constexpr (R == 2) return qd2; else return qd3;
  };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int blk = wave & (NB - 1);
  const bool pwave = wave < NB;
  const int hh = lane >> 5, l32 = lane & 31;
  const int G = a.Hq / a.Hkv;
  int kt, pair;
  decode_kv_major((int)blockIdx.x, a.nkt_kv, a.B * a.Hkv, kt, pair);
  const int b = pair / a.Hkv, hk = pair - (pair / a.Hkv) * a.Hkv;
  const int S = a.S;
  const int64_t *docb = a.doc + b * a.doc_sb;
  const float sl2 = a.sl2;
  const char *qbase = reinterpret_cast<const char *>(a.q.row(b, hk * G, 0));
  const char *gbase = reinterpret_cast<const char *>(a.dout.row(b, hk * G, 0));
  const int64_t rbase = ((int64_t)b * a.Hq + hk * G) * S;

  const int kv = kt * BN + blk * 32 + l32;
  const int kvr = kv < S ? kv : S - 1;
  const int64_t kvdoc = docb[kvr];
  bf16x8_t kvf[NDK];  // K (P-wave) or V (dP-wave) fragments of this lane's KV row
  {
    const bf16_t *row = pwave ? a.k.row(b, hk, kvr) : a.v.row(b, hk, kvr);
#pragma unroll
    for (int dk = 0; dk < NDK; ++dk)
      kvf[dk] = *reinterpret_cast<const bf16x8_t *>(row + 16 * dk + 8 * hh);
  }
  f32x16_t acc[NDB];  // dV (P-wave) or dK (dP-wave)
#pragma unroll
  for (int i = 0; i < NDB; ++i) acc[i] = zero16();

  // This thread's two 16-byte chunks of a swizzled 32-row sub-tile.  With
  // kept dS the two P-waves issue every Q / dO chunk (four each per operand:
  // chunk i * 128 + tid, rows 8 i + tid / 16, and the swizzle repeats every
  // 16 rows, so chunks i and i + 2 share a lane offset): the dP-waves, whose
  // dS stores share the in-order vmcnt, then never wait on a DMA.
  uint32_t qoff[NCH], goff[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    int r, c;
    SwzTile<DP>::at(DS ? i * 128 + (tid & 127) : i * NT + tid, r, c);
    qoff[i] = (uint32_t)((r * a.q.ss + c * 8) * 2);
    goff[i] = (uint32_t)((r * a.dout.ss + c * 8) * 2);
  }
  int roffs[NDK], coffs[NDB][2];
  {
    const int j = lane & 15, g = lane >> 4;
#pragma unroll
    for (int dk = 0; dk < NDK; ++dk) {
      roffs[dk] = SwzTile<DP>::off(l32, 16 * dk + 8 * hh);
      asm volatile("" : "+v"(roffs[dk]));
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int col = 32 * db + 16 * (g & 1) + 4 * (j & 3);
      const int row = 4 * hh + (j >> 2);
      coffs[db][0] = SwzTile<DP>::off(row, col);
      coffs[db][1] = SwzTile<DP>::off(row + 8, col);
      asm volatile("" : "+v"(coffs[db][0]), "+v"(coffs[db][1]));
    }
  }
  auto rfrag = [&](const char *t, int dk) {
    return *reinterpret_cast<const bf16x8_t *>(t + roffs[dk]);
  };
  auto cfrag = [&](const char *t, int f) {  // f = qk * NDB + db
    const char *base = t + (f / NDB) * 16 * DP * 2;
    const int db = f % NDB;
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base + coffs[db][0]));
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base + coffs[db][1]));
    typedef short i16x8_t __attribute__((ext_vector_type(8)));
    i16x8_t r = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return *reinterpret_cast<bf16x8_t *>(&r);
  };

  const int cnt = a.kcnt[b * a.nkt_kv + kt];
  const int T = G * 2 * cnt;  // steps: 32-row query sub-tile outer (last first), head inner
  {
    const int32_t *lst = a.klist + ((int64_t)b * a.nkt_kv + kt) * a.nqt_kv;
    for (int i = tid; i < T; i += NT) {
      const int u = 2 * cnt - 1 - i / G, g = i - (i / G) * G;
      const int e = lst[u >> 1];
      steps[i] = (plan_tile(e) * kQStep + 32 * (u & 1)) | (g << 20) | ((e & 3) << 28);
    }
  }
  auto step_info = [&](int t) {
    return __builtin_amdgcn_readfirstlane(steps[t < T ? t : T - 1]);
  };
  // One buffer resource per operand over this (pack, GQA group)'s rows; a
  // step's DMA passes its byte offset as the scalar offset (the host keeps
  // these extents below 2 GiB on this path).
  const auto qrs = buf_rsrc(qbase, kNoBound), grs = buf_rsrc(gbase, kNoBound);
  const auto lrs = buf_rsrc(a.lse + rbase, kNoBound), trs = buf_rsrc(a.delta + rbase, kNoBound);
  const auto drs = buf_rsrc(docb, kNoBound);
  const uint32_t qsh2 = (uint32_t)(a.q.sh * 2), qss2 = (uint32_t)(a.q.ss * 2);
  const uint32_t gsh2 = (uint32_t)(a.dout.sh * 2), gss2 = (uint32_t)(a.dout.ss * 2);
  auto dma_step = [&](int si, auto Rc) {
    const uint32_t q0 = si & 0xfffff, g = (si >> 20) & 0xff;
    const uint32_t ro = (g * (uint32_t)S + q0) * 4u;
    if (wave == 0 && lane < 8) dma16_rs(lrs, ro, 16 * lane, lslot(Rc));
    if (wave == 0 && lane >= 8 && lane < 16) dma16_rs(trs, ro, 16 * (lane - 8), lslot(Rc));
    if (wave == 1 && lane < 16) dma16_rs(drs, q0 * 8u, 16 * lane, dslot(Rc));
    const uint32_t qo = g * qsh2 + q0 * qss2, go = g * gsh2 + q0 * gss2;
    if constexpr (DS) {
      if (pwave) {
        // The LDS destinations are formed here, not hoisted out of the loop
        // (eight per slot would hold 32 SGPRs).
        int wb = wave * 1024;
        asm volatile("" : "+s"(wb));
#pragma unroll
        for (int i = 0; i < 2 * NCH; ++i)
          dma16_rs(qrs, qo + (i >> 1) * 16 * qss2, qoff[i & 1], qslot(Rc) + i * 2048 + wb);
#pragma unroll
        for (int i = 0; i < 2 * NCH; ++i)
          dma16_rs(grs, go + (i >> 1) * 16 * gss2, goff[i & 1], gslot(Rc) + i * 2048 + wb);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NCH; ++i) dma16_rs(qrs, qo, qoff[i], qslot(Rc) + (i * 4 + wave) * 1024);
#pragma unroll
      for (int i = 0; i < NCH; ++i) dma16_rs(grs, go, goff[i], gslot(Rc) + (i * 4 + wave) * 1024);
    }
  };
  const int kvmax = kt * BN + blk * 32 + 31;
  auto mask = [&](f32x16_t &sv, int si, const int64_t *qd) {
    const int q0 = si & 0xfffff, kind = si >> 28;
    const bool diag = q0 < kvmax;
    const int rel = kv - q0 - 4 * hh;
    if (kind == 2) {
      if (!diag) return;
#pragma unroll
      for (int j = 0; j < 16; ++j) sv[j] = rel <= 8 * (j >> 2) + (j & 3) ? sv[j] : -INFINITY;
      return;
    }
    int64_t dq[16];
    lds_docs16(qd, hh, dq);
    if (diag) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const bool ok = (rel <= 8 * (j >> 2) + (j & 3)) & (dq[j] == kvdoc);
        sv[j] = ok ? sv[j] : -INFINITY;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) sv[j] = dq[j] == kvdoc ? sv[j] : -INFINITY;
    }
  };
  auto load16 = [&](const float *p, float (&o)[16]) {
#pragma unroll
    for (int jg = 0; jg < 4; ++jg) {
      const float4 v = *reinterpret_cast<const float4 *>(p + 8 * jg + 4 * hh);
      o[4 * jg] = v.x; o[4 * jg + 1] = v.y; o[4 * jg + 2] = v.z; o[4 * jg + 3] = v.w;
    }
  };
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  auto put2 = [&](bf16x8_t (&f)[2], int j, float x0, float x1) {
    bf16x2_t pp;
    pp[0] = (bf16_t)x0;
    pp[1] = (bf16_t)x1;
    asm volatile("" ::"v"(*reinterpret_cast<uint32_t *>(&pp)));
    f[j >> 3][j & 7] = pp[0];
    f[j >> 3][(j & 7) + 1] = pp[1];
  };
  auto bf = [](bf16_t x) { return (float)x; };

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  // Slot 3 stands in for "step -1" of the dP-wave's first body: zeros.
  {
    const u32x4 z = {0u, 0u, 0u, 0u};
    for (int i = tid; i < HB / 16; i += NT) reinterpret_cast<u32x4 *>(qs3)[i] = z;
    if (tid < 16) reinterpret_cast<u32x4 *>(ld3)[tid] = z;
    u32x4 *p1 = &pbuf[1][0][0][0];
    for (int i = tid; i < NB * 2 * 64; i += NT) p1[i] = z;
  }
  __syncthreads();  // the step table
  if (T > 0) {
    dma_step(step_info(0), I0());
    dma_step(step_info(1), I1());
  }
  wait_vmcnt<0>();
  __syncthreads();
  // Q and dO chunks of one step per P-wave (issued after its lse/doc DMAs).
  constexpr int NDMA_STEP = DS ? 4 * NCH : 2 * NCH;

  if (pwave) {
    // ---------------------------------------------------------- P-wave
    int si = T > 0 ? step_info(0) : 0, si2 = T > 0 ? step_info(2) : 0;
    auto body = [&](auto Rc, int t) {
      constexpr int R = decltype(Rc)::value;
      using IR = std::integral_constant<int, R>;
      using IR2 = std::integral_constant<int, R + 2>;
      __builtin_amdgcn_sched_barrier(0);
      dma_step(si2, IR2());
      float lse[16];
      load16(lslot(IR()), lse);
      f32x16_t sc = zero16();
#pragma unroll
      for (int dk = 0; dk < NDK; ++dk) sc = mfma32(rfrag(qslot(IR()), dk), kvf[dk], sc);
      bf16x8_t gcol[NVF];
#pragma unroll
      for (int f = 0; f < NVF; ++f) gcol[f] = cfrag(gslot(IR()), f);
      if ((si >> 28) != 1) mask(sc, si, dslot(IR()));
      bf16x8_t pf[2];
#pragma unroll
      for (int j = 0; j < 16; j += 2)
        put2(pf, j, fast_exp2(fmaf(sc[j], sl2, -lse[j])), fast_exp2(fmaf(sc[j + 1], sl2, -lse[j + 1])));
      pbuf[t & 1][blk][0][lane] = *reinterpret_cast<const u32x4 *>(&pf[0]);
      pbuf[t & 1][blk][1][lane] = *reinterpret_cast<const u32x4 *>(&pf[1]);
      // dV += P(t)^T dO(t)
#pragma unroll
      for (int f = 0; f < NVF; ++f) acc[f % NDB] = mfma32(pf[f / NDB], gcol[f], acc[f % NDB]);
      si = step_info(t + 1);
      si2 = step_info(t + 3);
      __builtin_amdgcn_s_waitcnt(0xC07F);  // P(t) written (lgkmcnt(0))
      wait_vmcnt<NDMA_STEP>();
      block_sync_nofence();
    };
    int t = 0;
    for (; t + 4 <= T; t += 4) {
      body(I0(), t);
      body(I1(), t + 1);
      body(I2(), t + 2);
      body(I3(), t + 3);
    }
    if (t < T) { body(I0(), t); ++t; }
    if (t < T) { body(I1(), t); ++t; }
    if (t < T) { body(I2(), t); ++t; }
    wait_vmcnt<0>();
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int d = 32 * db + l32;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int kvw = kt * BN + blk * 32 + 8 * (j >> 2) + 4 * hh + (j & 3);
        if (kvw < S) a.dv.row(b, hk, kvw)[d] = (bf16_t)acc[db][j];
      }
    }
  } else {
    // ---------------------------------------------------------- dP-wave
    f32x16_t pc = zero16();  // dP(t-1); zero before the first step
    int si2 = T > 0 ? step_info(2) : 0;
    // Kept dS: this wave's 32 x 32 sub-block of step t-1 goes to its block
    // (query tile, this KV tile), head g, query half; lane (KV row l32, half
    // hh) writes its 16 query slots 16 hh .. 16 hh + 15 as two 16-byte stores.
    char *dsreg = nullptr;
    uint32_t dslane = 0;
    if constexpr (DS) {
      dsreg = a.ds + ((int64_t)b * a.Hkv + hk) * a.ds_pair;
      dslane = (uint32_t)(blk * G * 4096 + l32 * 64 + hh * 32);
    }
    auto store_ds = [&](int si, const bf16x8_t (&dsf)[2]) {
      const uint32_t q0 = si & 0xfffff, g = (si >> 20) & 0xff;
      const uint32_t qt = q0 >> 6, qs = (q0 >> 5) & 1;
      const uint32_t blkoff =
          (qt * (qt + 1) / 2 + (uint32_t)kt) * (uint32_t)(G * 8192) + (g * 2 + qs) * 2048u;
      char *p = dsreg + blkoff + dslane;
      __builtin_nontemporal_store(*reinterpret_cast<const u32x4 *>(&dsf[0]),
                                  reinterpret_cast<u32x4 *>(p));
      __builtin_nontemporal_store(*reinterpret_cast<const u32x4 *>(&dsf[1]),
                                  reinterpret_cast<u32x4 *>(p + 16));
    };
    auto body = [&](auto Rc, int t) {
      constexpr int R = decltype(Rc)::value;
      using IR = std::integral_constant<int, R>;
      using IRm1 = std::integral_constant<int, R + 3>;  // step t-1's slot
      using IR2 = std::integral_constant<int, R + 2>;
      __builtin_amdgcn_sched_barrier(0);
      dma_step(si2, IR2());
      // dP(t) = dO(t) V^T
      f32x16_t pn = zero16();
#pragma unroll
      for (int dk = 0; dk < NDK; ++dk) pn = mfma32(rfrag(gslot(IR()), dk), kvf[dk], pn);
      // dS(t-1) = P(t-1) (dP(t-1) - delta(t-1)); dK += dS(t-1)^T Q(t-1)
      float dlt[16];
      load16(lslot(IRm1()) + 32, dlt);
      bf16x8_t pp[2];
      *reinterpret_cast<u32x4 *>(&pp[0]) = pbuf[(t + 1) & 1][blk][0][lane];
      *reinterpret_cast<u32x4 *>(&pp[1]) = pbuf[(t + 1) & 1][blk][1][lane];
      bf16x8_t qcol[NVF];
#pragma unroll
      for (int f = 0; f < NVF; ++f) qcol[f] = cfrag(qslot(IRm1()), f);
      bf16x8_t dsf[2];
#pragma unroll
      for (int j = 0; j < 16; j += 2)
        put2(dsf, j, bf(pp[j >> 3][j & 7]) * (pc[j] - dlt[j]),
             bf(pp[j >> 3][(j & 7) + 1]) * (pc[j + 1] - dlt[j + 1]));
#pragma unroll
      for (int f = 0; f < NVF; ++f) acc[f % NDB] = mfma32(dsf[f / NDB], qcol[f], acc[f % NDB]);
      if constexpr (DS) {
        if (t > 0) store_ds(step_info(t - 1), dsf);
      }
      pc = pn;
      si2 = step_info(t + 3);
      // With kept dS this wave issues no DMA (the P-waves wait for it).
      if constexpr (!DS) wait_vmcnt<NDMA_STEP>();
      block_sync_nofence();
    };
    int t = 0;
    for (; t + 4 <= T; t += 4) {
      body(I0(), t);
      body(I1(), t + 1);
      body(I2(), t + 2);
      body(I3(), t + 3);
    }
    if (t < T) { body(I0(), t); ++t; }
    if (t < T) { body(I1(), t); ++t; }
    if (t < T) { body(I2(), t); ++t; }
    wait_vmcnt<0>();
    // Last step: dS(T-1) with P(T-1), written before the final barrier above.
    const int rl = T > 0 ? (T - 1) % 4 : 3;  // T == 0: the zeroed slot, a no-op
    const char *qt = rl == 0 ? qs0 : rl == 1 ? qs1 : rl == 2 ? qs2 : qs3;
    const float *lt = rl == 0 ? ld0 : rl == 1 ? ld1 : rl == 2 ? ld2 : ld3;
    float dlt[16];
    load16(lt + 32, dlt);
    bf16x8_t pp[2];
    *reinterpret_cast<u32x4 *>(&pp[0]) = pbuf[T > 0 ? (T - 1) & 1 : 1][blk][0][lane];
    *reinterpret_cast<u32x4 *>(&pp[1]) = pbuf[T > 0 ? (T - 1) & 1 : 1][blk][1][lane];
    bf16x8_t dsf[2];
#pragma unroll
    for (int j = 0; j < 16; j += 2)
      put2(dsf, j, bf(pp[j >> 3][j & 7]) * (pc[j] - dlt[j]),
           bf(pp[j >> 3][(j & 7) + 1]) * (pc[j + 1] - dlt[j + 1]));
#pragma unroll
    for (int f = 0; f < NVF; ++f) acc[f % NDB] = mfma32(dsf[f / NDB], cfrag(qt, f), acc[f % NDB]);
    if constexpr (DS) {
      if (T > 0) store_ds(step_info(T - 1), dsf);
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int d = 32 * db + l32;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int kvw = kt * BN + blk * 32 + 8 * (j >> 2) + 4 * hh + (j & 3);
        if (kvw < S) a.dk.row(b, hk, kvw)[d] = (bf16_t)(acc[db][j] * a.scale);
      }
    }
  }
}

// Split dK/dV: sum the fp32 partials of the G query heads of each KV head
// (and, for KV tiles whose list was walked in two halves, of both halves;
// fixed order, so the sums do not depend on scheduling).
// Element-wise form for views that do not allow 16-byte access.
__global__ __launch_bounds__(256) void attn_bwd_reduce_scalar(BwdArgs a) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)a.B * a.Hkv * a.S * a.D;
  if (t >= total) return;
  const int d = (int)(t % a.D);
  const int64_t sidx = (t / a.D) % a.S;
  const int hk = (int)((t / ((int64_t)a.D * a.S)) % a.Hkv);
  const int b = (int)(t / ((int64_t)a.D * a.S * a.Hkv));
  const int G = a.Hq / a.Hkv;
  const bool halves =
      a.kv_chunk > 0 && 2 * a.kcnt[b * a.nkt_kv + (int)(sidx / a.kv_tile)] >= a.kv_chunk;
  float sk = 0.f, sv = 0.f;
  for (int g = 0; g < G; ++g) {
    const int64_t o = (((int64_t)b * a.Hq + hk * G + g) * a.S + sidx) * a.D + d;
    sk += a.dk_part[o];
    sv += a.dv_part[o];
    if (halves) {
      sk += a.dk_part2[o];
      sv += a.dv_part2[o];
    }
  }
  a.dk.row(b, hk, sidx)[d] = (bf16_t)(sk * a.scale);
  a.dv.row(b, hk, sidx)[d] = (bf16_t)sv;
}

// Eight consecutive head-dim elements per thread (16-byte partial loads, one
// 16-byte store per output; D % 8 == 0, 16-byte aligned views and
// workspace); the row index (pack, KV head, position) is one 32-bit division
// by D / 8.  Same additions in the same order as the element-wise form.
__device__ __forceinline__ void kv_reduce_body(const BwdArgs &a, int block) {
  typedef float f32x4_t __attribute__((ext_vector_type(4)));
  const int t = block * 256 + (int)threadIdx.x;
  const int cpr = a.D >> 3;  // 8-element chunks per row
  const int rows = a.B * a.Hkv * a.S;
  const int row = t / cpr;
  if (row >= rows) return;
  const int d = (t - row * cpr) * 8;
  const int sidx = row % a.S, bh = row / a.S;
  const int hk = bh % a.Hkv, b = bh / a.Hkv;
  const int G = a.Hq / a.Hkv;
  const bool halves =
      a.kv_chunk > 0 && 2 * a.kcnt[b * a.nkt_kv + sidx / a.kv_tile] >= a.kv_chunk;
  f32x4_t k0 = {0.f, 0.f, 0.f, 0.f}, k1 = k0, v0 = k0, v1 = k0;
  const int64_t hstride = (int64_t)a.S * a.D;
  int64_t o = (((int64_t)b * a.Hq + hk * G) * a.S + sidx) * a.D + d;
  for (int g = 0; g < G; ++g, o += hstride) {
    k0 += *reinterpret_cast<const f32x4_t *>(a.dk_part + o);
    k1 += *reinterpret_cast<const f32x4_t *>(a.dk_part + o + 4);
    v0 += *reinterpret_cast<const f32x4_t *>(a.dv_part + o);
    v1 += *reinterpret_cast<const f32x4_t *>(a.dv_part + o + 4);
    if (halves) {
      k0 += *reinterpret_cast<const f32x4_t *>(a.dk_part2 + o);
      k1 += *reinterpret_cast<const f32x4_t *>(a.dk_part2 + o + 4);
      v0 += *reinterpret_cast<const f32x4_t *>(a.dv_part2 + o);
      v1 += *reinterpret_cast<const f32x4_t *>(a.dv_part2 + o + 4);
    }
  }
  bf16x8_t ok, ov;
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    ok[x] = (bf16_t)(k0[x] * a.scale);
    ok[x + 4] = (bf16_t)(k1[x] * a.scale);
    ov[x] = (bf16_t)v0[x];
    ov[x + 4] = (bf16_t)v1[x];
  }
  *reinterpret_cast<bf16x8_t *>(a.dk.row(b, hk, sidx) + d) = ok;
  *reinterpret_cast<bf16x8_t *>(a.dv.row(b, hk, sidx) + d) = ov;
}
__global__ __launch_bounds__(256) void attn_bwd_reduce(BwdArgs a) {
  kv_reduce_body(a, (int)blockIdx.x);
}

// ---------------------------------------------------------------- dQ
template <int DP, int WAVES>
__device__ __forceinline__ void dq_body(const BwdArgs &a) {
  constexpr int NT = 64 * WAVES;
  constexpr int BM = 32 * WAVES, BN = kKvStep;
  constexpr int KP = DP + 8;
  constexpr int NDK = DP / 16, NDB = DP / 32, CH = DP / 8;
  constexpr int NLD = BN * CH / NT;
  static_assert(NLD >= 1 && BN * CH % NT == 0, "tile/thread mismatch");
  __shared__ __align__(16) bf16_t Ks[BN * KP];
  __shared__ __align__(16) bf16_t Vs[BN * KP];
  __shared__ int64_t kdoc[BN];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hh = lane >> 5, l32 = lane & 31;
  int qt, b, h;
  decode_q_major((int)blockIdx.x, a.nqt_dq, a.B, a.Hq, a.Hkv, qt, b, h);
  const int hk = h / (a.Hq / a.Hkv);
  const bool vec = a.vec != 0;
  const int64_t *docb = a.doc + b * a.doc_sb;

  const int qi = qt * BM + wave * 32 + l32;
  const bool qvalid = qi < a.S;
  const int64_t qdoc = qvalid ? docb[qi] : 0;
  const int64_t row_o = ((int64_t)b * a.Hq + h) * a.S + (qvalid ? qi : 0);
  const float lse2 = qvalid ? a.lse[row_o] : 0.f;
  bf16x8_t qf[NDK], gf[NDK];
  float dlt = 0.f;
  {
    const int64_t r = qvalid ? qi : 0;
    const bf16_t *qrow = a.q.row(b, h, r), *grow = a.dout.row(b, h, r);
    const bf16_t *orow = a.o.row(b, h, r);
#pragma unroll
    for (int dk = 0; dk < NDK; ++dk) {
      qf[dk] = load_row8(qrow, 16 * dk + 8 * hh, a.D, qvalid, vec);
      gf[dk] = load_row8(grow, 16 * dk + 8 * hh, a.D, qvalid, vec);
      const bf16x8_t of = load_row8(orow, 16 * dk + 8 * hh, a.D, qvalid, vec);
#pragma unroll
      for (int i = 0; i < 8; ++i) dlt += (float)gf[dk][i] * (float)of[i];
    }
    // The two lane halves hold complementary 8-element slices of the row.
    dlt += __shfl_xor(dlt, 32);
    if (qvalid && hh == 0) a.delta[row_o] = dlt;
  }
  f32x16_t dq_acc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) dq_acc[i] = zero16();

  const int cnt = a.qcnt[b * a.nqt_dq + qt];
  const int32_t *lst = a.qlist + ((int64_t)b * a.nqt_dq + qt) * a.nkt_dq;
  bf16x8_t kr[NLD], vr[NLD];
  int64_t dr = 0;
  auto fetch = [&](int e) {
    const int kv0 = plan_tile(e) * BN;
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int c = tid + NT * i;
      const int row = c / CH, col = (c % CH) * 8;
      const int kvr = kv0 + row;
      const bool ok = kvr < a.S;
      kr[i] = load_row8(a.k.row(b, hk, ok ? kvr : 0), col, a.D, ok, vec);
      vr[i] = load_row8(a.v.row(b, hk, ok ? kvr : 0), col, a.D, ok, vec);
    }
    if (tid < BN) dr = (kv0 + tid < a.S) ? docb[kv0 + tid] : 0;
  };
  if (cnt > 0) fetch(lst[0]);
  for (int it = 0; it < cnt; ++it) {
    const int e = lst[it];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int c = tid + NT * i;
      const int row = c / CH, col = (c % CH) * 8;
      *reinterpret_cast<bf16x8_t *>(&Ks[row * KP + col]) = kr[i];
      *reinterpret_cast<bf16x8_t *>(&Vs[row * KP + col]) = vr[i];
    }
    if (tid < BN) kdoc[tid] = dr;
    __syncthreads();
    if (it + 1 < cnt) fetch(lst[it + 1]);

    const int kv0 = plan_tile(e) * BN;
    const bool full = plan_full(e);
    bf16x8_t dsf[4];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      f32x16_t sacc = zero16(), pacc = zero16();
#pragma unroll
      for (int dk = 0; dk < NDK; ++dk) {
        const int off = (32 * blk + l32) * KP + 16 * dk + 8 * hh;
        sacc = mfma32(*reinterpret_cast<const bf16x8_t *>(&Ks[off]), qf[dk], sacc);
        pacc = mfma32(*reinterpret_cast<const bf16x8_t *>(&Vs[off]), gf[dk], pacc);
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int kr_ = 32 * blk + 8 * (j >> 2) + 4 * hh + (j & 3);
        const int kvr = kv0 + kr_;
        const bool ok = full || (qvalid && kvr <= qi && kvr < a.S && kdoc[kr_] == qdoc);
        const float p = ok ? fast_exp2(fmaf(sacc[j], a.sl2, -lse2)) : 0.f;
        dsf[2 * blk + (j >> 3)][j & 7] = (bf16_t)(p * (pacc[j] - dlt));
      }
    }
    // dQ^T += K^T dS^T; A = K^T rows d, k slots kv = 16kk + pi(hh, s).
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        dq_acc[db] = mfma32(lds_col_frag(Ks, KP, 16 * kk, 32 * db, lane), dsf[kk], dq_acc[db]);
  }
  if (!qvalid) return;
  bf16_t *qrow = a.dq.row(b, h, qi);
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
      const int d0 = 32 * db + 8 * jq + 4 * hh;
#pragma unroll
      for (int x = 0; x < 4; ++x)
        if (d0 + x < a.D) qrow[d0 + x] = (bf16_t)(dq_acc[db][4 * jq + x] * a.scale);
    }
}

// ---------------------------------------------------------------- dQ (pipelined)
// Pipelined dQ (same eligibility as attn_bwd_dkdv_pipe).  Lane <-> query row
// as in the forward: Q and dO fragments in registers, D = rowsum(dO * O) from
// them (written for the dK/dV kernel).  The plan's KV tiles are walked as
// 32-row sub-tiles u; K, V and the KV documents arrive by DMA through a
// 4-slot ring of swizzled tiles (three sub-tiles in flight).  Body u issues
// the MFMAs of S(u+1)^T = K Q^T and dP(u+1)^T = V dO^T between the P/dS math
// of sub-tile u, then dQ^T += K^T dS^T with K^T as column fragments of the
// same K tile.  Head dim 64 fits two waves per SIMD (~214 registers); head
// dim 128 needs ~320 and runs one.
constexpr int kAheadDq = 1;  // K / V fragment reads in flight ahead of their MFMAs

// Two waves per SIMD where the registers allow it (D = 64, and D = 128 with
// 4-wave workgroups); the 2-wave D = 128 variant needs more and runs one.
template <int DP, int WAVES>
__global__ __launch_bounds__(64 * WAVES)
__attribute__((amdgpu_waves_per_eu(DP == 64 || WAVES == 4 ? 2 : 1, DP == 64 || WAVES == 4 ? 2 : 1)))
void attn_bwd_dq_pipe(BwdArgs a) {
  constexpr int NT = 64 * WAVES, BM = 32 * WAVES;
  constexpr int NDK = DP / 16, NDB = DP / 32;
  constexpr int HB = 32 * DP * 2;
  using Dma = TileDma<DP, 32, NT>;
  constexpr int NDMA = Dma::NDMA;
  constexpr int NVF = 2 * NDB;
  __shared__ __align__(16) char ks0[HB], ks1[HB], ks2[HB], ks3[HB];
  __shared__ __align__(16) char vs0[HB], vs1[HB], vs2[HB], vs3[HB];
  __shared__ __align__(16) int64_t kd0[32], kd1[32], kd2[32], kd3[32];
  auto kslot = [&](auto Rc) -> char * {
    constexpr int R = decltype(Rc)::value;
    if constexpr (R == 0) return ks0; else if constexpr (R == 1) return ks1;
    else if constexpr (R == 2) return ks2; else return ks3;
  };
  auto vslot = [&](auto Rc) -> char * {
    constexpr int R = decltype(Rc)::value;
    if constexpr (R == 0) return vs0; else if constexpr (R == 1) return vs1;
    else if constexpr (R == 2) return vs2; else return vs3;
  };
  auto dslot = [&](auto Rc) -> int64_t * {
    constexpr int R = decltype(Rc)::value;
    if constexpr (R == 0) return kd0; else if constexpr (R == 1) return kd1;
    else if constexpr (R == 2) return kd2; else return kd3;
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hh = lane >> 5, l32 = lane & 31;
  int qt, b, h;
  // Workgroup = (KV chunk, then the q-major order of the unsplit launch);
  // unused chunk slots exit at once.
  const int nbase = a.nqt_dq * a.B * a.Hq;
  const int split = (int)blockIdx.x / nbase;
  decode_q_major((int)blockIdx.x - split * nbase, a.nqt_dq, a.B, a.Hq, a.Hkv, qt, b, h);
  const int cnt_all = a.qcnt[b * a.nqt_dq + qt];
  int e_begin = 0, cnt = cnt_all;
  bool part = false;
  if (a.dq_chunk > 0) {
    const int nch = (cnt_all + a.dq_chunk - 1) / a.dq_chunk;
    if (split >= (nch > 0 ? nch : 1)) return;  // uniform over the workgroup
    e_begin = split * a.dq_chunk;
    cnt = min(a.dq_chunk, cnt_all - e_begin);
    part = nch > 1;
  }
  const int hk = h / (a.Hq / a.Hkv);
  const int S = a.S;
  const int64_t *docb = a.doc + b * a.doc_sb;
  const float sl2 = a.sl2;
  const char *Kb = reinterpret_cast<const char *>(a.k.row(b, hk, 0));
  const char *Vb = reinterpret_cast<const char *>(a.v.row(b, hk, 0));
  // One buffer resource per operand for the whole loop; a tile's DMA passes
  // its first row's byte offset as the scalar offset (the host keeps S * row
  // stride * 2 below 2 GiB on this path).
  const auto krs = buf_rsrc(Kb, 0x7fffffff), vrs = buf_rsrc(Vb, 0x7fffffff);
  const auto drs = buf_rsrc(docb, 0x7fffffff);
  const uint32_t kss2 = (uint32_t)(a.k.ss * 2), vss2 = (uint32_t)(a.v.ss * 2);

  const int qi = qt * BM + wave * 32 + l32;
  const bool qvalid = qi < S;
  const int qr = qvalid ? qi : S - 1;
  const int64_t qdoc = docb[qr];
  const int64_t row_o = ((int64_t)b * a.Hq + h) * S + qr;
  const float lse2 = a.lse[row_o];
  bf16x8_t qf[NDK], gf[NDK];
  float dlt = 0.f;
  {
    const bf16_t *qrow = a.q.row(b, h, qr), *grow = a.dout.row(b, h, qr);
    const bf16_t *orow = a.o.row(b, h, qr);
#pragma unroll
    for (int dk = 0; dk < NDK; ++dk) {
      qf[dk] = *reinterpret_cast<const bf16x8_t *>(qrow + 16 * dk + 8 * hh);
      gf[dk] = *reinterpret_cast<const bf16x8_t *>(grow + 16 * dk + 8 * hh);
      const bf16x8_t of = *reinterpret_cast<const bf16x8_t *>(orow + 16 * dk + 8 * hh);
#pragma unroll
      for (int i = 0; i < 8; ++i) dlt += (float)gf[dk][i] * (float)of[i];
    }
    dlt = xor32_sum(dlt);  // the lane halves hold complementary slices of the row
    if (qvalid && hh == 0 && split == 0) a.delta[row_o] = dlt;
  }
  f32x16_t dq_acc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) dq_acc[i] = zero16();

  uint32_t koff[NDMA], voff[NDMA];
  Dma::offsets(a.k.ss, wave, lane, koff);
  Dma::offsets(a.v.ss, wave, lane, voff);
  int roffs[NDK], coffs[NDB][2];
  {
    const int j = lane & 15, g = lane >> 4;
#pragma unroll
    for (int dk = 0; dk < NDK; ++dk) {
      roffs[dk] = SwzTile<DP>::off(l32, 16 * dk + 8 * hh);
      asm volatile("" : "+v"(roffs[dk]));
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int col = 32 * db + 16 * (g & 1) + 4 * (j & 3);
      const int row = 4 * hh + (j >> 2);
      coffs[db][0] = SwzTile<DP>::off(row, col);
      coffs[db][1] = SwzTile<DP>::off(row + 8, col);
      asm volatile("" : "+v"(coffs[db][0]), "+v"(coffs[db][1]));
    }
  }
  auto rfrag = [&](const char *t, int dk) {
    return *reinterpret_cast<const bf16x8_t *>(t + roffs[dk]);
  };
  auto cfrag = [&](const char *t, int f) {  // f = kk * NDB + db
    const char *base = t + (f / NDB) * 16 * DP * 2;
    const int db = f % NDB;
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base + coffs[db][0]));
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base + coffs[db][1]));
    typedef short i16x8_t __attribute__((ext_vector_type(8)));
    i16x8_t r = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return *reinterpret_cast<bf16x8_t *>(&r);
  };

  const int U = 2 * cnt;
  const int32_t *lst = a.qlist + ((int64_t)b * a.nqt_dq + qt) * a.nkt_dq + e_begin;
  auto entry = [&](int u) { return lst[(u < U ? u : U - 1) >> 1]; };
  auto row0 = [&](int e, int u) { return plan_tile(e) * kKvStep + 32 * (u & 1); };
  // (The row is passed in, not computed here: calling another lambda inside
  // this generic lambda's DMA address makes clang drop the kernel's stub.)
  auto dma_sub = [&](int kv0, auto Rc) {
    if (wave == 0 && lane < 16) dma16_rs(drs, (uint32_t)kv0 * 8u, 16 * lane, dslot(Rc));
    Dma::copy_rs(krs, (uint32_t)kv0 * kss2, koff, kslot(Rc), wave);
    Dma::copy_rs(vrs, (uint32_t)kv0 * vss2, voff, vslot(Rc), wave);
  };
  // Element mask of a PARTIAL sub-tile: same document and kv <= q.
  // Tests and shortcuts as in attn_fwd_pipe (query rows past the sequence end
  // are left unmasked: their dQ is never stored).
  const int qmin = qt * BM + wave * 32;
  auto mask = [&](f32x16_t &sv, int e, int kv0, const int64_t *kd) {
    const bool diag = kv0 + 31 > qmin;
    const int rel = qi - kv0 - 4 * hh;
    if (plan_causal(e)) {
      if (!diag) return;
#pragma unroll
      for (int j = 0; j < 16; ++j) sv[j] = 8 * (j >> 2) + (j & 3) <= rel ? sv[j] : -INFINITY;
      return;
    }
    int64_t dkv[16];
    lds_docs16(kd, hh, dkv);
    if (diag) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const bool ok = (8 * (j >> 2) + (j & 3) <= rel) & (dkv[j] == qdoc);
        sv[j] = ok ? sv[j] : -INFINITY;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) sv[j] = dkv[j] == qdoc ? sv[j] : -INFINITY;
    }
  };
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  auto ds2 = [&](int j, const f32x16_t &sc, const f32x16_t &pc, bf16x8_t (&dsf)[2]) {
    bf16x2_t dd;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float p = fast_exp2(fmaf(sc[j + i], sl2, -lse2));
      dd[i] = (bf16_t)(p * (pc[j + i] - dlt));
    }
    asm volatile("" ::"v"(*reinterpret_cast<uint32_t *>(&dd)));
    dsf[j >> 3][j & 7] = dd[0];
    dsf[j >> 3][(j & 7) + 1] = dd[1];
  };

  if (U > 0) {
    int ew[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ew[i] = entry(i + 1);
    const int e0 = entry(0);
    dma_sub(row0(e0, 0), I0());
    dma_sub(row0(ew[0], 1), I1());
    dma_sub(row0(ew[1], 2), I2());
    wait_vmcnt<0>();
    __syncthreads();
    f32x16_t sc = zero16(), pc = zero16();
#pragma unroll
    for (int dk = 0; dk < NDK; ++dk) {
      sc = mfma32(rfrag(ks0, dk), qf[dk], sc);
      pc = mfma32(rfrag(vs0, dk), gf[dk], pc);
    }
    if (!plan_full(e0)) mask(sc, e0, row0(e0, 0), kd0);

    auto body = [&](auto Rc, int u) {
      constexpr int R = decltype(Rc)::value;
      using IR = std::integral_constant<int, R>;
      using IR1 = std::integral_constant<int, (R + 1) % 4>;
      using IR3 = std::integral_constant<int, (R + 3) % 4>;
      const int e1 = __builtin_amdgcn_readfirstlane(ew[0]);
      const int e3 = __builtin_amdgcn_readfirstlane(ew[2]);
      const int e4 = entry(u + 5);
      __builtin_amdgcn_sched_barrier(0);
      dma_sub(row0(e3, u + 3), IR3());
      // K / V row fragments of sub-tile u+1 stream kAheadDq steps ahead of
      // their MFMAs (holding all of them costs 64 registers at D = 128).
      bf16x8_t ka[NDK], va[NDK];
#pragma unroll
      for (int dk = 0; dk < kAheadDq; ++dk) {
        ka[dk] = rfrag(kslot(IR1()), dk);
        va[dk] = rfrag(vslot(IR1()), dk);
      }
      f32x16_t sn = zero16(), pn = zero16();
      bf16x8_t dsf[2];
      __builtin_amdgcn_sched_barrier(0);
      constexpr int JPS = 16 / NDK;
      constexpr int FPS = (NVF + NDK - 1) / NDK;  // K^T fragments read per head-dim step
      bf16x8_t kcol[NVF];
#pragma unroll
      for (int dk = 0; dk < NDK; ++dk) {
        if (dk + kAheadDq < NDK) {
          ka[dk + kAheadDq] = rfrag(kslot(IR1()), dk + kAheadDq);
          va[dk + kAheadDq] = rfrag(vslot(IR1()), dk + kAheadDq);
        }
        sn = mfma32(ka[dk], qf[dk], sn);
        pn = mfma32(va[dk], gf[dk], pn);
#pragma unroll
        for (int j = dk * JPS; j < (dk + 1) * JPS; j += 2) ds2(j, sc, pc, dsf);
#pragma unroll
        for (int f = dk * FPS; f < (dk + 1) * FPS && f < NVF; ++f) kcol[f] = cfrag(kslot(IR()), f);
        // dQ^T += K^T dS^T for the first half of dS (complete after step
        // NDK/2 - 1) in the second half of the steps, next to S and dP.
        if constexpr (NVF == NDK) {
          if (dk >= NDK / 2 && dk - NDK / 2 < NDB) {
            const int f = dk - NDK / 2;
            dq_acc[f % NDB] = mfma32(kcol[f], dsf[0], dq_acc[f % NDB]);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // The rest of dQ^T += K^T dS^T (A = K^T: column fragments of the K
      // tile, read during the loop above).
#pragma unroll
      for (int f = (NVF == NDK ? NDB : 0); f < NVF; ++f)
        dq_acc[f % NDB] = mfma32(kcol[f], dsf[f / NDB], dq_acc[f % NDB]);
      sc = sn;
      pc = pn;
      if (!plan_full(e1)) mask(sc, e1, row0(e1, u + 1), dslot(IR1()));
      wait_vmcnt<2 * NDMA>();
      block_sync_nofence();
      ew[0] = ew[1];
      ew[1] = ew[2];
      ew[2] = ew[3];
      ew[3] = e4;
    };
    int u = 0;
    for (; u + 4 < U; u += 4) {
      body(I0(), u);
      body(I1(), u + 1);
      body(I2(), u + 2);
      body(I3(), u + 3);
    }
    if (u + 1 < U) { body(I0(), u); ++u; }
    if (u + 1 < U) { body(I1(), u); ++u; }
    if (u + 1 < U) { body(I2(), u); ++u; }
    wait_vmcnt<0>();
    const int rl = u & 3;
    const char *kt = rl == 0 ? ks0 : rl == 1 ? ks1 : rl == 2 ? ks2 : ks3;
    bf16x8_t dsf[2];
#pragma unroll
    for (int j = 0; j < 16; j += 2) ds2(j, sc, pc, dsf);
#pragma unroll
    for (int f = 0; f < NVF; ++f)
      dq_acc[f % NDB] = mfma32(cfrag(kt, f), dsf[f / NDB], dq_acc[f % NDB]);
  }

  if (!qvalid) return;
  if (part) {
    // This chunk's unscaled dQ rows, fp32 (summed and scaled by attn_bwd_dq_reduce).
    const int64_t prow = (((int64_t)split * a.B + b) * a.Hq + h) * S + qi;
    float *pq = a.dq_part + prow * DP;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) {
        typedef float f32x4_t __attribute__((ext_vector_type(4)));
        f32x4_t o4;
#pragma unroll
        for (int x = 0; x < 4; ++x) o4[x] = dq_acc[db][4 * jq + x];
        *reinterpret_cast<f32x4_t *>(pq + 32 * db + 8 * jq + 4 * hh) = o4;
      }
    return;
  }
  bf16_t *qrow = a.dq.row(b, h, qi);
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
      typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
      bf16x4_t o4;
#pragma unroll
      for (int x = 0; x < 4; ++x) o4[x] = (bf16_t)(dq_acc[db][4 * jq + x] * a.scale);
      *reinterpret_cast<bf16x4_t *>(qrow + 32 * db + 8 * jq + 4 * hh) = o4;
    }
}

// dQ of split query tiles = scale * sum of the chunk partials (bf16): DP/4
// threads per (pack, head, query row), four elements each; rows of unsplit
// tiles were written by attn_bwd_dq_pipe and are skipped.
template <int DP>
__device__ __forceinline__ void dq_reduce_body(const BwdArgs &a, int bm, int block) {
  constexpr int TPR = DP / 4, RPB = 256 / TPR;
  typedef float f32x4_t __attribute__((ext_vector_type(4)));
  const int64_t row = (int64_t)block * RPB + threadIdx.x / TPR;
  const int d0 = (threadIdx.x % TPR) * 4;
  const int64_t rows = (int64_t)a.B * a.Hq * a.S;
  if (row >= rows) return;
  const int q = (int)(row % a.S);
  const int64_t bh = row / a.S;
  const int h = (int)(bh % a.Hq), b = (int)(bh / a.Hq);
  const int cnt = a.qcnt[b * a.nqt_dq + q / bm];
  const int nch = (cnt + a.dq_chunk - 1) / a.dq_chunk;
  if (nch <= 1) return;
  const float *pq = a.dq_part + row * DP + d0;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int c = 0; c < nch; ++c) acc += *reinterpret_cast<const f32x4_t *>(pq + c * rows * DP);
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  bf16x4_t o4;
#pragma unroll
  for (int x = 0; x < 4; ++x) o4[x] = (bf16_t)(acc[x] * a.scale);
  *reinterpret_cast<bf16x4_t *>(a.dq.row(b, h, q) + d0) = o4;
}
template <int DP>
__global__ __launch_bounds__(256) void attn_bwd_dq_reduce(BwdArgs a, int bm) {
  dq_reduce_body<DP>(a, bm, (int)blockIdx.x);
}
// Both reductions in one launch (the split dK/dV sums in the first kv_blocks
// workgroups, the dQ sums in the rest): they are independent, and a launch
// of a few microseconds of work costs about as much again to start.
template <int DP>
__global__ __launch_bounds__(256) void attn_bwd_reduce_both(BwdArgs a, int bm, int kv_blocks) {
  if ((int)blockIdx.x < kv_blocks) kv_reduce_body(a, (int)blockIdx.x);
  else dq_reduce_body<DP>(a, bm, (int)blockIdx.x - kv_blocks);
}

// Two entry points over one body: two waves per SIMD (so one wave's softmax
// overlaps the other's MFMAs) wherever the registers fit without spilling.
template <int DP, int WAVES>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(2, 2))) void
attn_bwd_dq(BwdArgs a) {
  dq_body<DP, WAVES>(a);
}

template <int DP, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void attn_bwd_dq_wide(BwdArgs a) {
  dq_body<DP, WAVES>(a);
}

// ---------------------------------------------------------------- kept-dS dQ
// D = rowsum(dO * O) for the kept-dS backward (there the dK/dV kernel runs
// first and no dQ kernel forms D on the way).  DP / 8 lanes per row,
// kDeltaRowsPerGroup rows per lane group, all loads issued before the sums,
// non-temporal (dO and O are streamed once; at cfg3 185 -> 179 us with four
// rows instead of eight, 221 -> 185 us non-temporal instead of cached).
constexpr int kDeltaRowsPerGroup = 4;
template <int DP>
__global__ __launch_bounds__(256) void attn_bwd_delta(BwdArgs a) {
  constexpr int TPR = DP / 8, RPP = 256 / TPR, NP = kDeltaRowsPerGroup;
  const int64_t rows = (int64_t)a.B * a.Hq * a.S;
  const int sub = threadIdx.x % TPR;
  u32x4 gv[NP], ov[NP];
  int64_t r[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    r[p] = ((int64_t)blockIdx.x * NP + p) * RPP + threadIdx.x / TPR;
    if (r[p] < rows) {
      const int s = (int)(r[p] % a.S);
      const int64_t bh = r[p] / a.S;
      const int h = (int)(bh % a.Hq), b = (int)(bh / a.Hq);
      gv[p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(a.dout.row(b, h, s) + 8 * sub));
      ov[p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(a.o.row(b, h, s) + 8 * sub));
    }
  }
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    float dot = 0.f;
    if (r[p] < rows) {
      const bf16_t *ge = reinterpret_cast<const bf16_t *>(&gv[p]);
      const bf16_t *oe = reinterpret_cast<const bf16_t *>(&ov[p]);
#pragma unroll
      for (int i = 0; i < 8; ++i) dot += (float)ge[i] * (float)oe[i];
    }
#pragma unroll
    for (int m = TPR / 2; m >= 1; m >>= 1) dot += __shfl_xor(dot, m, TPR);
    if (r[p] < rows && sub == 0) a.delta[r[p]] = dot;
  }
}

// dQ = scale * dS K over the kept dS blocks (AttnConfig::ds, head dim 128).
// One workgroup per (pack, four query heads of one GQA group, 64-row query
// tile): wave w owns head 4 quad + w / 2 and query half w % 2, accumulating
// dQ^T = K^T dS^T (lane <-> query slot, 4 x 16 registers <-> head dim) over
// the tile's plan list, one 32-row KV half per step.  Per step the K half
// (8 KiB, swizzled) and the eight dS sub-blocks of the quad at that KV half
// (16 KiB, contiguous in HBM) arrive by LDS DMA through a 3-slot ring; both
// operands are read with ds_read_b64_tr_b16 (K^T columns as in the dQ
// kernel, dS^T columns from the 32 x 32 sub-blocks at a 64-byte pitch), so
// the k slots of both follow pi.  No recomputation: one MFMA product per
// pair where the dQ kernel runs three, and the kernel streams the dS blocks
// (2 bytes per pair and head) from HBM.
constexpr int kDsMaxTiles = kPairsMaxSteps / 8;  // 64-row KV tiles per list (G >= 4)

template <int DP>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4)))
void attn_bwd_dq_ds(BwdArgs a) {
  static_assert(DP == 128, "head dim 128");
  constexpr int NT = 512, NDB = DP / 32;
  constexpr int KB = 32 * DP * 2;  // one 32-row K half
  constexpr int SB = 8 * 2048;     // 4 heads x 2 query halves of 32 x 32 bf16
  constexpr int64_t kNoBound = 0x7fffffff;
  using Dma = TileDma<DP, 32, NT>;
  static_assert(Dma::NDMA == 1, "one K chunk per thread");
  __shared__ __align__(16) char ks0[KB], ks1[KB], ks2[KB];
  __shared__ __align__(16) char ss0[SB], ss1[SB], ss2[SB];
  __shared__ int32_t ents[kDsMaxTiles];
  auto kslot = [&](auto Rc) -> char * {
    constexpr int R = decltype(Rc)::value;
    if constexpr (R == 0) return ks0; else if constexpr (R == 1) return ks1; else return ks2;
  };
  auto sslot = [&](auto Rc) -> char * {
    constexpr int R = decltype(Rc)::value;
    if constexpr (R == 0) return ss0; else if constexpr (R == 1) return ss1; else return ss2;
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gg = wave >> 1, qs = wave & 1;
  const int hh = lane >> 5;
  const int G = a.Hq / a.Hkv, nquad = a.Hq / 4, nqt = a.nqt_dq;
  // Grid: (pack, quad) pairs spread over the 8 XCDs (workgroup i runs on XCD
  // i % 8), each XCD walking its pairs' query tiles late first, so the
  // workgroups resident on one XCD read the same KV head's K halves from its L2.
  int qt, pr;
  {
    const int bid = (int)blockIdx.x, npairs = a.B * nquad;
    if (npairs % 8 == 0) {
      const int x = bid & 7, j = bid >> 3;
      pr = (j / nqt) * 8 + x;
      qt = nqt - 1 - (j - (j / nqt) * nqt);
    } else {
      pr = bid / nqt;
      qt = nqt - 1 - (bid - pr * nqt);
    }
  }
  const int b = pr / nquad, quad = pr - (pr / nquad) * nquad;
  const int h0 = 4 * quad, hk = h0 / G, g0 = h0 - hk * G;
  const int h = h0 + gg;
  const int cnt = a.qcnt[b * nqt + qt];
  const int U = 2 * cnt;  // 32-row KV halves
  {
    const int32_t *lst = a.qlist + ((int64_t)b * nqt + qt) * a.nkt_dq;
    for (int i = tid; i < cnt; i += NT) ents[i] = lst[i];
  }
  const char *Kb = reinterpret_cast<const char *>(a.k.row(b, hk, 0));
  const auto krs = buf_rsrc(Kb, kNoBound);
  const auto drs = buf_rsrc(a.ds + ((int64_t)b * a.Hkv + hk) * a.ds_pair, kNoBound);
  const uint32_t kss2 = (uint32_t)(a.k.ss * 2);
  const uint32_t tri = (uint32_t)(qt * (qt + 1) / 2);
  const uint32_t blkb = (uint32_t)(G * 8192), halfb = (uint32_t)(G * 4096), quadb = (uint32_t)(g0 * 4096);
  uint32_t koff[1];
  Dma::offsets(a.k.ss, wave, lane, koff);
  const uint32_t soff0 = (uint32_t)((wave * 64 + lane) * 16), soff1 = soff0 + 8 * 1024;
  // ds_read_b64_tr_b16 addresses (see lds_col_frag): K^T of head-dim block
  // db (swizzled K half), dS^T of this wave's sub-block (64-byte pitch).
  int coffs[NDB][2], soffs[2];
  {
    const int j = lane & 15, g = lane >> 4;
    const int row = 4 * hh + (j >> 2);
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int col = 32 * db + 16 * (g & 1) + 4 * (j & 3);
      coffs[db][0] = SwzTile<DP>::off(row, col);
      coffs[db][1] = SwzTile<DP>::off(row + 8, col);
      asm volatile("" : "+v"(coffs[db][0]), "+v"(coffs[db][1]));
    }
    const int col = 16 * (g & 1) + 4 * (j & 3);
    soffs[0] = (gg * 2 + qs) * 2048 + (row * 32 + col) * 2;
    soffs[1] = soffs[0] + 8 * 64;
    asm volatile("" : "+v"(soffs[0]), "+v"(soffs[1]));
  }
  auto trd = [](const char *p0, const char *p1) {
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)p0);
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)p1);
    typedef short i16x8_t __attribute__((ext_vector_type(8)));
    i16x8_t r = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return *reinterpret_cast<bf16x8_t *>(&r);
  };
  auto dma_sub = [&](int u, auto Rc) {
    const int uu = u < U ? u : U - 1;
    const int e = __builtin_amdgcn_readfirstlane(ents[uu >> 1]);
    const uint32_t kt = (uint32_t)plan_tile(e), half = (uint32_t)(uu & 1);
    Dma::copy_rs(krs, (kt * 64 + half * 32) * kss2, koff, kslot(Rc), wave);
    const uint32_t so = (tri + kt) * blkb + half * halfb + quadb;
    dma16_rs_nt(drs, so, soff0, sslot(Rc) + wave * 1024);
    dma16_rs_nt(drs, so, soff1, sslot(Rc) + (8 + wave) * 1024);
  };
  f32x16_t acc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) acc[i] = zero16();
  __syncthreads();  // the list
  if (U > 0) {
    dma_sub(0, I0());
    dma_sub(1, I1());
    wait_vmcnt<3>();
    __syncthreads();
    auto body = [&](auto Rc, int u) {
      constexpr int R = decltype(Rc)::value;
      using IR2 = std::integral_constant<int, (R + 2) % 3>;
      __builtin_amdgcn_sched_barrier(0);
      dma_sub(u + 2, IR2());
      const char *kt = kslot(Rc), *st = sslot(Rc);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8_t bfr = trd(st + soffs[0] + ks * 16 * 64, st + soffs[1] + ks * 16 * 64);
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const char *kb = kt + ks * 16 * DP * 2;
          acc[db] = mfma32(trd(kb + coffs[db][0], kb + coffs[db][1]), bfr, acc[db]);
        }
      }
      wait_vmcnt<3>();
      block_sync_nofence();
    };
    int u = 0;
    for (; u + 3 <= U; u += 3) {
      body(I0(), u);
      body(I1(), u + 1);
      body(I2(), u + 2);
    }
    if (u < U) { body(I0(), u); ++u; }
    if (u < U) { body(I1(), u); ++u; }
    wait_vmcnt<0>();
  }
  // Lane <-> query slot sl (row 8 (sl % 16 / 4) + 4 (sl / 16) + sl % 4 of the
  // query half), register j <-> head-dim row 8 (j / 4) + 4 hh + j % 4.
  const int sl = lane & 31;
  const int q = qt * 64 + qs * 32 + 8 * ((sl & 15) >> 2) + 4 * (sl >> 4) + (sl & 3);
  bf16_t *qrow = a.dq.row(b, h, q);
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
      typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
      bf16x4_t o4;
#pragma unroll
      for (int x = 0; x < 4; ++x) o4[x] = (bf16_t)(acc[db][4 * jq + x] * a.scale);
      *reinterpret_cast<bf16x4_t *>(qrow + 32 * db + 8 * jq + 4 * hh) = o4;
    }
}

View view_of(const pb_bhsd *t) {
  View v;
  v.p = static_cast<bf16_t *>(t->data);
  v.sb = t->stride_b;
  v.sh = t->stride_h;
  v.ss = t->stride_s;
  return v;
}

}  // namespace attn
}  // namespace pb

extern "C" int pb_attn_config(int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t d,
                              int64_t *out) {
  using namespace pb::attn;
  pb::clear_error();
  if (b < 1 || hq < 1 || hkv < 1 || s < 1 || d < 1 || hq % hkv) {
    pb::set_error("pb_attn_config: bad shape");
    return PB_EINVAL;
  }
  const AttnConfig c = attn_config(b, hq, hkv, s, d);
  out[0] = c.fwd_q_tile();
  out[1] = kKvStep;
  out[2] = kQStep;
  out[3] = c.kv_tile();
  out[4] = c.dq_q_tile();
  out[5] = kKvStep;
  out[6] = attn_bwd_workspace(b, hq, hkv, s, d);
  out[7] = c.split;
  out[8] = attn_fwd_workspace(b, hq, hkv, s, d);
  out[9] = c.fwd_chunk;
  return PB_OK;
}

extern "C" int pb_attn_bwd(const pb_bhsd *q, const pb_bhsd *k, const pb_bhsd *v,
                           const pb_bhsd *out, const pb_bhsd *dout, const pb_bhsd *dq,
                           const pb_bhsd *dk, const pb_bhsd *dv, const float *lse,
                           void *workspace, const int64_t *doc_ids, int64_t doc_stride,
                           const int32_t *q_plan_counts, const int32_t *q_plan_lists,
                           const int32_t *kv_plan_counts, const int32_t *kv_plan_lists,
                           int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t d, float scale,
                           int dtype, void *stream) {
  using namespace pb;
  using namespace pb::attn;
  clear_error();
  int rc = check_attn_shape("pb_attn_bwd", b, hq, hkv, s, d, dtype);
  if (rc) return rc;
  PB_CHECK_ARG(scale > 0.f, "pb_attn_bwd: softmax scale must be positive");
  PB_CHECK_ARG(q && k && v && out && dout && dq && dk && dv && lse && workspace && doc_ids &&
                   q_plan_counts && q_plan_lists && kv_plan_counts && kv_plan_lists,
               "pb_attn_bwd: null argument");
  const AttnConfig cfg = attn_config(b, hq, hkv, s, d);
  BwdArgs a;
  a.q = view_of(q); a.k = view_of(k); a.v = view_of(v); a.o = view_of(out);
  a.dout = view_of(dout); a.dq = view_of(dq); a.dk = view_of(dk); a.dv = view_of(dv);
  a.lse = lse;
  char *ws = static_cast<char *>(workspace);
  a.delta = reinterpret_cast<float *>(ws);
  const int64_t delta_bytes = (b * hq * s * 4 + 255) / 256 * 256;
  a.dk_part = reinterpret_cast<float *>(ws + delta_bytes);
  a.dv_part = a.dk_part + b * hq * s * d;
  a.dk_part2 = a.dv_part + b * hq * s * d;
  a.dv_part2 = a.dk_part2 + b * hq * s * d;
  a.kv_chunk = 0;
  a.kv_tile = (int)cfg.kv_tile();
  a.dq_chunk = 0;
  a.dq_part = reinterpret_cast<float *>(ws + attn_bwd_dq_part_offset(b, hq, s, d, cfg.split != 0));
  a.ds = nullptr;
  a.ds_pair = 0;
  a.doc = doc_ids;
  a.doc_sb = doc_stride;
  a.qcnt = q_plan_counts; a.qlist = q_plan_lists;
  a.kcnt = kv_plan_counts; a.klist = kv_plan_lists;
  a.B = (int)b; a.Hq = (int)hq; a.Hkv = (int)hkv; a.S = (int)s; a.D = (int)d;
  a.nqt_dq = (int)((s + cfg.dq_q_tile() - 1) / cfg.dq_q_tile());
  a.nkt_dq = (int)((s + kKvStep - 1) / kKvStep);
  a.nqt_kv = (int)((s + kQStep - 1) / kQStep);
  a.nkt_kv = (int)((s + cfg.kv_tile() - 1) / cfg.kv_tile());
  a.sl2 = scale * kLog2e;
  a.scale = scale;
  a.vec = views_vectorizable(d, {q, k, v, out, dout, dq, dk, dv});
  hipStream_t st = as_stream(stream);
  // dq first: it also writes delta = rowsum(dO * O), which dkdv reads.
  dim3 g_q((unsigned)(a.nqt_dq * b * hq));
  dim3 g_kv((unsigned)(a.nkt_kv * b * hkv * (cfg.split ? hq / hkv : 1)));
#define PB_DQ(DP, W)                                                                \
  do {                                                                              \
    if (DP == 128 && W == 2)                                                        \
      hipLaunchKernelGGL((attn_bwd_dq_wide<DP, W>), g_q, dim3(64 * W), 0, st, a);   \
    else                                                                            \
      hipLaunchKernelGGL((attn_bwd_dq<DP, W>), g_q, dim3(64 * W), 0, st, a);        \
  } while (0)
#define PB_KV(DP, W, SP) hipLaunchKernelGGL((attn_bwd_dkdv<DP, W, SP>), g_kv, dim3(64 * W), 0, st, a)
#define PB_BY_D(M, ...) \
  do { if (d <= 32) M(32, __VA_ARGS__); else if (d <= 64) M(64, __VA_ARGS__); else M(128, __VA_ARGS__); } while (0)
  // DMA-pipelined kernels where views, documents and the sequence length allow.
  const bool pipe = a.vec && (d == 64 || d == 128) && s % 64 == 0 &&
                    (reinterpret_cast<uintptr_t>(doc_ids) & 15) == 0 && doc_stride % 2 == 0 &&
                    (reinterpret_cast<uintptr_t>(lse) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(workspace) & 15) == 0 &&
                    32 * std::max({q->stride_s, dout->stride_s, k->stride_s, v->stride_s}) <
                        (1LL << 30) &&
                    s * std::max(k->stride_s, v->stride_s) * 2 < (1LL << 31) &&
                    ((hq / hkv - 1) * std::max(q->stride_h, dout->stride_h) +
                     s * std::max(q->stride_s, dout->stride_s)) * 2 < (1LL << 31) &&
                    (hq / hkv) * s * 4 < (1LL << 31) && s * 8 < (1LL << 31);
  // The paired kernel addresses one (pack, GQA group)'s Q / dO rows, and its
  // lse / delta rows, with 32-bit byte offsets.
  const int64_t G = hq / hkv;
  const bool pairs_fit =
      ((G - 1) * std::max(q->stride_h, dout->stride_h) + s * std::max(q->stride_s, dout->stride_s)) *
              2 < (1LL << 31) &&
      G * s * 4 < (1LL << 31);
  const bool pairs = pipe && cfg.pairs && G * s / 32 <= kPairsMaxSteps && pairs_fit;
  if (pairs && cfg.ds) {
    // Kept dS: D, then dK/dV storing dS, then dQ = scale * dS K.
    a.ds = ws + delta_bytes;
    a.ds_pair = ds_pair_bytes(G, s);
    const int64_t rows = b * hq * s;
    const int64_t drows = (int64_t)kDeltaRowsPerGroup * (256 / (128 / 8));  // rows per workgroup
    hipLaunchKernelGGL(attn_bwd_delta<128>, dim3((unsigned)((rows + drows - 1) / drows)), dim3(256),
                       0, st, a);
    rc = launch_status("pb_attn_bwd(delta)");
    if (rc) return rc;
    hipLaunchKernelGGL((attn_bwd_dkdv_pairs<128, true>), g_kv, dim3(256), 0, st, a);
    rc = launch_status("pb_attn_bwd(dkdv)");
    if (rc) return rc;
    hipLaunchKernelGGL(attn_bwd_dq_ds<128>, dim3((unsigned)(b * (hq / 4) * a.nqt_dq)), dim3(512), 0,
                       st, a);
    return launch_status("pb_attn_bwd(dq)");
  }
  if (pipe && cfg.dq_chunk > 0) {
    a.dq_chunk = cfg.dq_chunk;
    g_q.x *= (unsigned)cfg.dq_splits;
  }
  if (pipe) {
#define PB_DQP(DP, W) hipLaunchKernelGGL((attn_bwd_dq_pipe<DP, W>), g_q, dim3(64 * W), 0, st, a)
    if (cfg.dq_waves == 4) { if (d == 128) PB_DQP(128, 4); else PB_DQP(64, 4); }
    else { if (d == 128) PB_DQP(128, 2); else PB_DQP(64, 2); }
#undef PB_DQP
  } else if (cfg.dq_waves == 4) PB_BY_D(PB_DQ, 4);
  else PB_BY_D(PB_DQ, 2);
  rc = launch_status("pb_attn_bwd(dq)");
  if (rc) return rc;
  if (pipe) {
#define PB_KVP(DP, W, SP) \
  hipLaunchKernelGGL((attn_bwd_dkdv_pipe<DP, W, SP>), g_kv, dim3(64 * W), 0, st, a)
    if (pairs)
      hipLaunchKernelGGL((attn_bwd_dkdv_pairs<128, false>), g_kv, dim3(256), 0, st, a);
    else if (cfg.kv_waves == 4) { if (d == 128) PB_KVP(128, 4, false); else PB_KVP(64, 4, false); }
    else if (cfg.split) {
      // Lists of >= kKvChunkSteps steps are walked as two halves by two workgroups.
      a.kv_chunk = kKvChunkSteps;
      g_kv.x *= 2;
      if (d == 128) PB_KVP(128, 2, true); else PB_KVP(64, 2, true);
    }
    else { if (d == 128) PB_KVP(128, 2, false); else PB_KVP(64, 2, false); }
#undef PB_KVP
  } else if (cfg.kv_waves == 4) PB_BY_D(PB_KV, 4, false);
  else if (cfg.split) PB_BY_D(PB_KV, 2, true);
  else PB_BY_D(PB_KV, 2, false);
#undef PB_BY_D
#undef PB_KV
#undef PB_DQ
  rc = launch_status("pb_attn_bwd(dkdv)");
  if (rc) return rc;
  const int64_t n8 = b * hkv * s * (d / 8);  // thread count of the 16-byte dK/dV reduce
  const bool kv_vec = cfg.split && a.vec && (reinterpret_cast<uintptr_t>(workspace) & 15) == 0 &&
                      n8 < (1LL << 31) - 256;
  const int64_t rows = b * hq * s, rpb = 256 / (d / 4);
  const int64_t q_blocks = a.dq_chunk > 0 ? (rows + rpb - 1) / rpb : 0;
  if (kv_vec && q_blocks > 0) {
    const int64_t kv_blocks = (n8 + 255) / 256;
    const dim3 grid((unsigned)(kv_blocks + q_blocks));
    if (d == 128)
      hipLaunchKernelGGL(attn_bwd_reduce_both<128>, grid, dim3(256), 0, st, a, cfg.dq_q_tile(),
                         (int)kv_blocks);
    else
      hipLaunchKernelGGL(attn_bwd_reduce_both<64>, grid, dim3(256), 0, st, a, cfg.dq_q_tile(),
                         (int)kv_blocks);
    return launch_status("pb_attn_bwd");
  }
  if (kv_vec) {
    hipLaunchKernelGGL(attn_bwd_reduce, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, st, a);
  } else if (cfg.split) {
    const int64_t n = b * hkv * s * d;
    hipLaunchKernelGGL(attn_bwd_reduce_scalar, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       a);
  }
  if (q_blocks > 0) {
    const dim3 rgrid((unsigned)q_blocks);
    if (d == 128) hipLaunchKernelGGL(attn_bwd_dq_reduce<128>, rgrid, dim3(256), 0, st, a, cfg.dq_q_tile());
    else hipLaunchKernelGGL(attn_bwd_dq_reduce<64>, rgrid, dim3(256), 0, st, a, cfg.dq_q_tile());
  }
  return launch_status("pb_attn_bwd");
}
