// Document-masked GQA attention forward for gfx950 (bf16 in, fp32 accumulate).
//
// Reference: the FlexAttention forward that packbalance/model/attention.py:98-122
// runs with the document BlockMask (mask doc[q] == doc[kv] && q >= kv, GQA
// query head h -> KV head h / (Hq/Hkv), scale 1/sqrt(D)).
//
// Work decomposition: one workgroup per (pack, query head, query tile of
// 32*W rows) with W = 2 or 4 waves of 32 query rows each (AttnConfig picks W
// from the grid size).  The workgroup walks only the KV tiles (64 rows) that
// the tile plan lists for its query tile -- tiles with no same-document causal
// pair are never loaded -- and applies the element mask only on PARTIAL tiles.
// On small grids the pipelined kernel also splits each list into chunks of
// fwd_chunk tiles (one workgroup each, attn_config); a query tile with more
// than one chunk writes per-chunk fp32 outputs and log-sum-exps, and
// attn_fwd_combine merges them (o = sum_c 2^(lse_c - lse) o_c,
// lse = log2 sum_c 2^lse_c).
//
// Per KV tile a wave computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16, so a
// lane owns one query column: the online-softmax max/sum are lane-local plus
// one exchange with lane^32, and the O^T accumulator of a lane belongs to a
// single query (one rescale factor per lane).  P^T leaves the accumulators as
// the B operand of O^T += V^T P^T directly (see attn_common.hpp for the k-slot
// permutation), so P never touches LDS; V^T fragments come from the
// transposing LDS load ds_read_b64_tr_b16.
//
// Two kernels share this scheme: attn_fwd_pipe (16-byte aligned views, head
// dim 64 or 128, sequence a multiple of 64: DMA-fed swizzled LDS rings and a
// software-pipelined body, described below) and attn_fwd_generic (everything
// else: K/V staged through registers into padded LDS tiles, element-wise
// loads where 16-byte access is not allowed).
#include <algorithm>
#include <type_traits>

#include "attn_common.hpp"

namespace pb {
namespace attn {

struct FwdArgs {
  const bf16_t *q;
  int64_t q_sb, q_sh, q_ss;
  const bf16_t *k;
  int64_t k_sb, k_sh, k_ss;
  const bf16_t *v;
  int64_t v_sb, v_sh, v_ss;
  bf16_t *o;
  int64_t o_sb, o_sh, o_ss;
  float *lse;  // [B][Hq][S], log2 domain of the scaled scores
  const int64_t *doc;
  int64_t doc_sb;
  const int32_t *cnt;   // [B][nqt]
  const int32_t *list;  // [B][nqt][nkt]
  int B, Hq, Hkv, S, D, nqt, nkt;
  float sl2;  // softmax scale * log2(e)
  int vec;    // 16-byte global access allowed
  // KV split (pipelined kernel): chunk = KV tiles per workgroup (0: whole
  // list); bm = query rows per tile; partial outputs [split][B][Hq][S][D]
  // and log-sum-exps [split][B][Hq][S], fp32.
  int chunk, bm;
  float *part_o, *part_lse;
};

// Generic path: any head dim <= 128, any strides / alignment (element-wise
// loads where 16-byte access is not allowed), K/V staged through registers.
template <int DP, int WAVES>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_fwd_generic(FwdArgs a) {
  constexpr int NT = 64 * WAVES;
  constexpr int BM = 32 * WAVES, BN = kKvStep;
  constexpr int KP = DP + 8;  // K / V row pitch in LDS (elements)
  constexpr int NDK = DP / 16;
  constexpr int NDB = DP / 32;
  constexpr int CH = DP / 8;              // 16-byte chunks per K/V row
  constexpr int NLD = BN * CH / NT;       // chunks per thread per tile
  static_assert(NLD >= 1 && BN * CH % NT == 0, "tile/thread mismatch");
  __shared__ __align__(16) bf16_t Ks[BN * KP];
  __shared__ __align__(16) bf16_t Vs[BN * KP];
  __shared__ int64_t kdoc[BN];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hh = lane >> 5, l32 = lane & 31;

  int qt, b, h;
  decode_q_major((int)blockIdx.x, a.nqt, a.B, a.Hq, a.Hkv, qt, b, h);
  const int hk = h / (a.Hq / a.Hkv);
  const int q0 = qt * BM;

  const bf16_t *Qb = a.q + b * a.q_sb + h * a.q_sh;
  const bf16_t *Kb = a.k + b * a.k_sb + hk * a.k_sh;
  const bf16_t *Vb = a.v + b * a.v_sb + hk * a.v_sh;
  const int64_t *docb = a.doc + b * a.doc_sb;
  const bool vec = a.vec != 0;

  const int qi = q0 + wave * 32 + l32;
  const bool qvalid = qi < a.S;
  const int64_t qdoc = qvalid ? docb[qi] : 0;
  bf16x8_t qf[NDK];
  {
    const bf16_t *qrow = Qb + (int64_t)(qvalid ? qi : 0) * a.q_ss;
#pragma unroll
    for (int dk = 0; dk < NDK; ++dk) qf[dk] = load_row8(qrow, 16 * dk + 8 * hh, a.D, qvalid, vec);
  }

  f32x16_t oacc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) oacc[i] = zero16();
  float m = -INFINITY, l = 0.f;

  const int cnt = a.cnt[b * a.nqt + qt];
  const int32_t *lst = a.list + ((int64_t)b * a.nqt + qt) * a.nkt;

  bf16x8_t kr[NLD], vr[NLD];
  int64_t dr = 0;
  auto fetch = [&](int e) {
    const int kv0 = plan_tile(e) * BN;
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int c = tid + NT * i;
      const int row = c / CH, col = (c % CH) * 8;
      const int kv = kv0 + row;
      const bool ok = kv < a.S;
      const int64_t r = ok ? kv : 0;
      kr[i] = load_row8(Kb + r * a.k_ss, col, a.D, ok, vec);
      vr[i] = load_row8(Vb + r * a.v_ss, col, a.D, ok, vec);
    }
    if (tid < BN) dr = (kv0 + tid < a.S) ? docb[kv0 + tid] : 0;
  };

  if (cnt > 0) fetch(lst[0]);
  for (int it = 0; it < cnt; ++it) {
    const int e = lst[it];
    __syncthreads();  // every wave is done reading the previous tile
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

    // S^T = K Q^T for the two 32-row halves of the tile.
    f32x16_t sacc[2];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      sacc[blk] = zero16();
#pragma unroll
      for (int dk = 0; dk < NDK; ++dk) {
        const bf16x8_t ka =
            *reinterpret_cast<const bf16x8_t *>(&Ks[(32 * blk + l32) * KP + 16 * dk + 8 * hh]);
        sacc[blk] = mfma32(ka, qf[dk], sacc[blk]);
      }
    }
    const int kv0 = plan_tile(e) * BN;
    const bool full = plan_full(e);
    // Running max kept in the log2-scaled domain; the per-element scale is
    // folded into the exp2 argument (one FMA per score).
    float mloc = -INFINITY;
    if (!full) {
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int kr_ = 32 * blk + 8 * (j >> 2) + 4 * hh + (j & 3);
          const int kv = kv0 + kr_;
          const bool ok = qvalid && kv <= qi && kv < a.S && kdoc[kr_] == qdoc;
          sacc[blk][j] = ok ? sacc[blk][j] : -INFINITY;
        }
    }
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int j = 0; j < 16; ++j) mloc = fmaxf(mloc, sacc[blk][j]);
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32)) * a.sl2;
    const float m_new = fmaxf(m, mloc);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = fast_exp2(m - m_use);
    m = m_new;
    l *= alpha;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int j = 0; j < 16; ++j) oacc[db][j] *= alpha;

    bf16x8_t pf[4];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float p = fast_exp2(fmaf(sacc[blk][j], a.sl2, -m_use));
        l += p;
        pf[2 * blk + (j >> 3)][j & 7] = (bf16_t)p;
      }

    // O^T += V^T P^T; A = V^T rows d, k slots kv = 16kk + pi(hh, s), read
    // from the row-major V tile with the transposing LDS load.
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        oacc[db] = mfma32(lds_col_frag(Vs, KP, 16 * kk, 32 * db, lane), pf[kk], oacc[db]);
  }

  const float l_tot = l + __shfl_xor(l, 32);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  if (qvalid) {
    bf16_t *orow = a.o + b * a.o_sb + (int64_t)qi * a.o_ss + h * a.o_sh;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) {
        const int d0 = 32 * db + 8 * jq + 4 * hh;
        if (vec && d0 + 4 <= a.D) {
          typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
          bf16x4_t o4;
#pragma unroll
          for (int x = 0; x < 4; ++x) o4[x] = (bf16_t)(oacc[db][4 * jq + x] * inv);
          *reinterpret_cast<bf16x4_t *>(orow + d0) = o4;
        } else {
#pragma unroll
          for (int x = 0; x < 4; ++x)
            if (d0 + x < a.D) orow[d0 + x] = (bf16_t)(oacc[db][4 * jq + x] * inv);
        }
      }
    if (hh == 0)
      a.lse[((int64_t)b * a.Hq + h) * a.S + qi] =
          l_tot > 0.f ? m + fast_log2(l_tot) : -INFINITY;
  }
}

// Pipelined path (16-byte aligned views and documents, D == DP in {64, 128},
// sequence length a multiple of 64).
//
// A wave owns MQ query rows (NQB = MQ/32 column blocks of S^T; each K / V
// fragment read from LDS feeds NQB MFMAs).  The launch uses MQ = 32, two
// waves per SIMD: MQ = 64 halves the LDS reads per MFMA but needs ~400
// registers, one wave per SIMD and AGPR<->VGPR copies, and measured slower
// (2.34 vs 1.94 ms on 8 x 8192-token packs, 32/8 heads, D 128).
// The KV tiles of the plan are walked as 32-row sub-tiles u.  K and V
// sub-tiles are copied global -> LDS by DMA (buffer_load_dwordx4 ... lds) into
// the swizzled layout, through 3-slot rings (slot = u % 3, compile-time in the
// 3x unrolled loop), one barrier per sub-tile.  Body u issues the DMA of
// K(u+3) and V(u+1), then runs a three-stage software pipeline over the DP/16
// head-dim steps: step k issues the k-th MFMA of S(u+1) = K(u+1) Q^T, the
// k-th MFMA of O^T += V(u-1)^T P(u-1)^T (P of the previous sub-tile, kept in
// registers) and a fixed slice of the exponentials of S(u), in that order
// (sched_barrier fences keep the compiler from regrouping them).  Every step
// thus pairs two MFMAs with an even share of the VALU work, and no MFMA
// waits for a result of its own body.  The running max moves only when a
// sub-tile's max exceeds it by more than kTau (log2 units), so P stays below
// 2^kTau and the exponentials are taken against the running max the body
// starts with; the body ends with a test of the lane sums that sends the
// rare sub-tile that moves a max (and a lane's first) down a wave-uniform
// slow path: the max, the O rescale (after PV(u-1), which was relative to the
// old max) and the exponentials again.  The body waits only for the DMA it
// issued.
template <int DP, int MQ, int WAVES>
__global__ __launch_bounds__(64 * WAVES)
__attribute__((amdgpu_waves_per_eu(MQ == 64 ? 1 : 2, MQ == 64 ? 1 : 2)))
void attn_fwd_pipe(FwdArgs a) {
  constexpr int NT = 64 * WAVES, NQB = MQ / 32, BM = MQ * WAVES;
  constexpr int NDK = DP / 16, NDB = DP / 32;
  constexpr int HB = 32 * DP * 2;  // bytes of one 32-row sub-tile
  using Dma = TileDma<DP, 32, NT>;
  constexpr int NDMA = Dma::NDMA;
  constexpr float kTau = 8.0f;
  // Softmax schedule over the NDK steps: the 8*NQB exponential pairs of
  // S(u), pair p in step p NDK / NPAIR (the max is only taken on the rare
  // slow path at the end of the body).
  constexpr int NPAIR = 8 * NQB;
  constexpr int NVF = 2 * NDB;  // V fragments per sub-tile: one PV MFMA per step
  static_assert(NDK >= 4 && NVF == NDK, "head dim");
  constexpr int kAhead = 4;  // steps whose K / V fragments are read before the first MFMA
  // Ring slots are separate LDS objects so that the compiler can tell a
  // fragment read of one slot from the DMA still in flight into another (it
  // would otherwise wait for all outstanding DMA before every read).
  __shared__ __align__(16) char ks0[HB], ks1[HB], ks2[HB];
  __shared__ __align__(16) char vs0[HB], vs1[HB], vs2[HB];
  __shared__ __align__(16) int64_t kd0[32], kd1[32], kd2[32];
  auto kslot = [&](auto Rc) -> char * {
    if constexpr (decltype(Rc)::value == 0) return ks0;
    else if constexpr (decltype(Rc)::value == 1) return ks1;
    else return ks2;
  };
  auto vslot = [&](auto Rc) -> char * {
    if constexpr (decltype(Rc)::value == 0) return vs0;
    else if constexpr (decltype(Rc)::value == 1) return vs1;
    else return vs2;
  };
  auto dslot = [&](auto Rc) -> int64_t * {
    if constexpr (decltype(Rc)::value == 0) return kd0;
    else if constexpr (decltype(Rc)::value == 1) return kd1;
    else return kd2;
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hh = lane >> 5, l32 = lane & 31;
  int qt, b, h;
  // Workgroup = (KV chunk, then the q-major order of the unsplit launch): the
  // first chunks of every list start first, unused chunk slots exit at once.
  const int nbase = a.nqt * a.B * a.Hq;
  const int split = (int)blockIdx.x / nbase;
  decode_q_major((int)blockIdx.x - split * nbase, a.nqt, a.B, a.Hq, a.Hkv, qt, b, h);
  const int cnt_all = a.cnt[b * a.nqt + qt];
  int e_begin = 0, cnt = cnt_all;
  bool part = false;
  if (a.chunk > 0) {
    const int nch = (cnt_all + a.chunk - 1) / a.chunk;
    if (split >= (nch > 0 ? nch : 1)) return;  // uniform over the workgroup
    e_begin = split * a.chunk;
    cnt = min(a.chunk, cnt_all - e_begin);
    part = nch > 1;
  }
  const int hk = h / (a.Hq / a.Hkv);
  const int S = a.S;
  const char *Kb = reinterpret_cast<const char *>(a.k + b * a.k_sb + hk * a.k_sh);
  const char *Vb = reinterpret_cast<const char *>(a.v + b * a.v_sb + hk * a.v_sh);
  const int64_t *docb = a.doc + b * a.doc_sb;
  const float sl2 = a.sl2;
  // One buffer resource per operand for the whole loop; a sub-tile's DMA
  // passes its first row's byte offset as the scalar offset (the host keeps
  // S * row stride * 2 below 2 GiB on this path).
  const auto krs = buf_rsrc(Kb, (int64_t)S * a.k_ss * 2);
  const auto vrs = buf_rsrc(Vb, (int64_t)S * a.v_ss * 2);
  const auto drs = buf_rsrc(docb, (int64_t)S * 8);
  const uint32_t kss2 = (uint32_t)(a.k_ss * 2), vss2 = (uint32_t)(a.v_ss * 2);

  uint32_t koff[NDMA], voff[NDMA];
  Dma::offsets(a.k_ss, wave, lane, koff);
  Dma::offsets(a.v_ss, wave, lane, voff);
  // Per-lane byte offsets of the fragments within a sub-tile: K row
  // fragments (row l32, columns 16dk + 8hh) and the two transposing reads of
  // a V column fragment (rows 4hh + j/4 and +8, column 32db + ...); rows
  // 16..31 repeat the swizzle of rows 0..15 at +16 * DP * 2 bytes.  Kept in
  // registers for the whole loop (the empty asm stops rematerialisation).
  int koffs[NDK], voffs[NDB][2];
  {
    const int j = lane & 15, g = lane >> 4;
#pragma unroll
    for (int dk = 0; dk < NDK; ++dk) {
      koffs[dk] = SwzTile<DP>::off(l32, 16 * dk + 8 * hh);
      asm volatile("" : "+v"(koffs[dk]));
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int col = 32 * db + 16 * (g & 1) + 4 * (j & 3);
      const int row = 4 * hh + (j >> 2);
      voffs[db][0] = SwzTile<DP>::off(row, col);
      voffs[db][1] = SwzTile<DP>::off(row + 8, col);
      asm volatile("" : "+v"(voffs[db][0]), "+v"(voffs[db][1]));
    }
  }
  auto kfrag = [&](const char *kt, int dk) {
    return *reinterpret_cast<const bf16x8_t *>(kt + koffs[dk]);
  };
  auto vfrag_of = [&](int f, const char *vt) {  // f = kk * NDB + db
    const char *base = vt + (f / NDB) * 16 * DP * 2;
    const int db = f % NDB;
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base + voffs[db][0]));
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base + voffs[db][1]));
    typedef short i16x8_t __attribute__((ext_vector_type(8)));
    i16x8_t r = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return *reinterpret_cast<bf16x8_t *>(&r);
  };

  // This lane's query rows (one per 32-column block), documents, Q fragments.
  int qi[NQB];
  bool qv[NQB];
  int64_t qdoc[NQB];
  bf16x8_t qf[NQB][NDK];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    qi[qb] = qt * BM + wave * MQ + qb * 32 + l32;
    qv[qb] = qi[qb] < S;
    const int qr = qv[qb] ? qi[qb] : S - 1;
    qdoc[qb] = docb[qr];
    const bf16_t *qrow = a.q + b * a.q_sb + h * a.q_sh + (int64_t)qr * a.q_ss;
#pragma unroll
    for (int dk = 0; dk < NDK; ++dk)
      qf[qb][dk] = *reinterpret_cast<const bf16x8_t *>(qrow + 16 * dk + 8 * hh);
  }

  f32x16_t oacc[NQB][NDB];
  float m_run[NQB], l_run[NQB];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    m_run[qb] = -INFINITY;
    l_run[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db) oacc[qb][db] = zero16();
  }

  const int U = 2 * cnt;  // 32-row sub-tiles
  const int32_t *lst = a.list + ((int64_t)b * a.nqt + qt) * a.nkt + e_begin;
  // Plan entry of sub-tile u (clamped to the last one).  Loaded one body
  // ahead and ahead of that body's DMA, so waiting for it never waits for
  // DMA (vmcnt counts in issue order).
  auto entry = [&](int u) { return lst[(u < U ? u : U - 1) >> 1]; };
  auto row0 = [&](int e, int u) { return plan_tile(e) * kKvStep + 32 * (u & 1); };

  // Element mask of a non-FULL sub-tile (kv rows kv0 .. kv0+31): same
  // document and kv <= q, as bitwise tests (no per-element branch).  Two
  // wave-uniform shortcuts: a sub-tile wholly at or before the wave's first
  // query row needs no causal test, and a CAUSAL plan tile no document test.
  // Rows past the sequence end are left unmasked: they are never stored.
  // kv0 + pi_row(hh, j) <= q  <=>  8(j/4) + j%4 <= q - kv0 - 4hh.
  const int qmin = qt * BM + wave * MQ;
  auto mask = [&](f32x16_t (&sv)[NQB], int e, int kv0, const int64_t *kd) {
    const bool diag = kv0 + 31 > qmin;
    int rel[NQB];
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) rel[qb] = qi[qb] - kv0 - 4 * hh;
    if (plan_causal(e)) {
      if (!diag) return;
#pragma unroll
      for (int j = 0; j < 16; ++j)
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb)
          sv[qb][j] = 8 * (j >> 2) + (j & 3) <= rel[qb] ? sv[qb][j] : -INFINITY;
      return;
    }
    int64_t dkv[16];
    lds_docs16(kd, hh, dkv);
    if (diag) {
#pragma unroll
      for (int j = 0; j < 16; ++j)
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
          const bool ok = (8 * (j >> 2) + (j & 3) <= rel[qb]) & (dkv[j] == qdoc[qb]);
          sv[qb][j] = ok ? sv[qb][j] : -INFINITY;
        }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j)
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) sv[qb][j] = dkv[j] == qdoc[qb] ? sv[qb][j] : -INFINITY;
    }
  };

  // Softmax state.  The exponentials of S(u) are taken against the running
  // max as it stands when the body starts (m_use: m_run, or 0 while it is
  // -inf), so they need no max of S(u) first.  That is exact whenever the max
  // would not have moved, i.e. every element is at most m_run + kTau, and the
  // lane's sum lt <= 2^kTau is a sufficient test of that (elements are
  // non-negative).  lim = 2^kTau, or -1 while m_run is -inf (no element seen:
  // the test fails, so a lane's first elements always take the slow path).
  // A wave in which some lane fails it takes the slow path at commit: the
  // max of S(u), the move rule (max > m_run + kTau), and, if a lane moved,
  // the O / l rescale and the exponentials again against the new max.
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  constexpr float kLim = 256.0f;  // 2^kTau
  static_assert(kTau == 8.0f, "kLim is 2^kTau");
  float m_use[NQB], lim[NQB], lt[NQB];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    m_use[qb] = 0.f;
    lim[qb] = -1.f;
  }
  // Exponential pair p of S(u) against m_use (j = 2 (p % 8) in block p / 8).
  // The row sum takes the fp32 values (as the reference's softmax does); only
  // the PV operand is rounded to bf16.
  auto exp_pair = [&](int p, const f32x16_t (&sv)[NQB], bf16x8_t (&pf)[NQB][2]) {
    const int qb = p / 8, j = 2 * (p % 8);
    const float p0 = fast_exp2(fmaf(sv[qb][j], sl2, -m_use[qb]));
    const float p1 = fast_exp2(fmaf(sv[qb][j + 1], sl2, -m_use[qb]));
    lt[qb] = j == 0 ? p0 + p1 : lt[qb] + (p0 + p1);
    bf16x2_t pp;
    pp[0] = (bf16_t)p0;
    pp[1] = (bf16_t)p1;
    pf[qb][j >> 3][j & 7] = pp[0];
    pf[qb][j >> 3][(j & 7) + 1] = pp[1];
    return pp;
  };
  // Slice `step` of the softmax of S(u): the exponential pairs spread evenly
  // over the NDK steps.  Each step's results pass through an empty volatile
  // asm, so they are computed inside the step (between the MFMAs it is
  // paired with) instead of being sunk towards their first use.
  auto softmax_step = [&](int step, const f32x16_t (&sv)[NQB], bf16x8_t (&pf)[NQB][2]) {
#pragma unroll
    for (int p = 0; p < NPAIR; ++p) {
      if (p * NDK / NPAIR != step) continue;
      bf16x2_t pp = exp_pair(p, sv, pf);
      asm volatile("" ::"v"(*reinterpret_cast<uint32_t *>(&pp)), "v"(lt[p / 8]));
    }
  };
  // End of sub-tile u (after PV(u-1), which used the old max): the rare slow
  // path, then the sums.
  auto softmax_commit = [&](const f32x16_t (&sv)[NQB], bf16x8_t (&pf)[NQB][2]) {
    bool slow = false;
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) slow |= !(lt[qb] <= lim[qb]);
    if (__builtin_expect(__builtin_amdgcn_ballot_w64(slow) != 0, 0)) {
      bool moved = false;
      float m_new[NQB];
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        float m0 = sv[qb][0];
#pragma unroll
        for (int j = 1; j < 16; ++j) m0 = fmaxf(m0, sv[qb][j]);
        const float m1 = xor32_max(m0) * sl2;
        const bool nq = m1 > m_run[qb] + kTau;
        moved |= nq;
        m_new[qb] = nq ? m1 : m_run[qb];
      }
      if (__builtin_amdgcn_ballot_w64(moved) != 0) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
          // Lanes whose max did not move keep alpha = 1 (their max may still
          // be -inf, where the difference would be NaN).
          const float alpha = m_new[qb] == m_run[qb] ? 1.f : fast_exp2(m_run[qb] - m_new[qb]);
          l_run[qb] *= alpha;
#pragma unroll
          for (int db = 0; db < NDB; ++db) oacc[qb][db] *= alpha;
          m_run[qb] = m_new[qb];
          m_use[qb] = m_new[qb] == -INFINITY ? 0.f : m_new[qb];
          lim[qb] = m_new[qb] == -INFINITY ? -1.f : kLim;
        }
#pragma unroll
        for (int p = 0; p < NPAIR; ++p) exp_pair(p, sv, pf);
      }
    }
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) l_run[qb] += lt[qb];
  };
  auto pv_step = [&](int f, const bf16x8_t &vf, const bf16x8_t (&pf)[NQB][2]) {
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb)
      oacc[qb][f % NDB] = mfma32(vf, pf[qb][f / NDB], oacc[qb][f % NDB]);
  };

  // kdoc of sub-tile rows kv0..kv0+31 into a ring slot: one DMA instruction
  // by 16 lanes of wave 0 (issued for every sub-tile, read for PARTIAL ones).
  auto load_kdoc = [&](int kv0, int64_t *dst) {
    if (wave == 0 && lane < 16) dma16_rs(drs, (uint32_t)kv0 * 8u, 16 * lane, dst);
  };

  f32x16_t sc[NQB];
  if (U > 0) {
    // Prologue: K(0..2), V(0) and their documents, then S(0).  U >= 2.
    int ew[4];  // entries of sub-tiles u+1 .. u+4 for body u (see below)
#pragma unroll
    for (int i = 0; i < 4; ++i) ew[i] = entry(i + 1);
    auto prefetch = [&](auto Rc, int u) {
      const int e = entry(u);
      load_kdoc(row0(e, u), dslot(Rc));
      Dma::copy_rs(krs, (uint32_t)row0(e, u) * kss2, koff, kslot(Rc), wave);
      if (decltype(Rc)::value == 0) Dma::copy_rs(vrs, (uint32_t)row0(e, u) * vss2, voff, vslot(Rc), wave);
    };
    prefetch(I0(), 0);
    prefetch(I1(), 1);
    prefetch(I2(), 2);  // repeats sub-tile 1 when U == 2
    wait_vmcnt<0>();
    __syncthreads();
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) sc[qb] = zero16();
#pragma unroll
    for (int dk = 0; dk < NDK; ++dk) {
      const bf16x8_t kf = kfrag(ks0, dk);
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) sc[qb] = mfma32(kf, qf[qb][dk], sc[qb]);
    }
    {
      const int e = entry(0);
      if (!plan_full(e)) mask(sc, e, row0(e, 0), kd0);
    }
    // The running max starts at S(0)'s (what the slow path would set), so the
    // first body's exponentials need no second pass.
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
      float m0 = sc[qb][0];
#pragma unroll
      for (int j = 1; j < 16; ++j) m0 = fmaxf(m0, sc[qb][j]);
      const float m1 = xor32_max(m0) * sl2;
      m_run[qb] = m1;
      m_use[qb] = m1 == -INFINITY ? 0.f : m1;
      lim[qb] = m1 == -INFINITY ? -1.f : kLim;
    }
    __syncthreads();  // K slot 0 is refilled by body 0

    // P(u-1) between bodies (the first body has no previous sub-tile).
    bf16x8_t pfp[NQB][2];
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) pfp[qb][0] = pfp[qb][1] = bf16x8_t{};

    // Body u (u + 1 < U), ring slot R = u % 3; PV = false for u = 0 only.
    // Every body issues the same DMA (past the last sub-tile, entry() repeats
    // it into a slot nobody reads any more), so the number of operations in
    // flight -- and the vmcnt to wait for -- is the same in every body.
    // Slots in body u: K(u+3) -> R (K(u) was read in body u-1), K(u+1) read
    // from R+1; V(u+1) -> R+1 (V(u-2) was read in body u-1), V(u-1) read from
    // R+2; documents of u+3 -> R, of u+1 read from R+1.
    auto body = [&](auto Rc, auto PVc, int u, f32x16_t (&sc)[NQB], f32x16_t (&sn)[NQB]) {
      constexpr int R = decltype(Rc)::value;
      constexpr int R1 = (R + 1) % 3, R2 = (R + 2) % 3;
      constexpr bool PV = decltype(PVc)::value;
      const int e1 = __builtin_amdgcn_readfirstlane(ew[0]);
      const int e3 = __builtin_amdgcn_readfirstlane(ew[2]);
      const int e4 = entry(u + 5);  // for body u + 1, issued before this body's DMA
      __builtin_amdgcn_sched_barrier(0);
      using IR = std::integral_constant<int, R>;
      using IR1 = std::integral_constant<int, R1>;
      using IR2 = std::integral_constant<int, R2>;
      load_kdoc(row0(e3, u + 3), dslot(IR()));
      Dma::copy_rs(krs, (uint32_t)row0(e3, u + 3) * kss2, koff, kslot(IR()), wave);
      Dma::copy_rs(vrs, (uint32_t)row0(e1, u + 1) * vss2, voff, vslot(IR1()), wave);
      // Fragments in the order the steps consume them: steps 0 .. kAhead-1
      // before the first MFMA, step k + kAhead during step k, so at most 12
      // LDS reads are outstanding and each MFMA waits only for its own
      // operands (the LGKM counter tracks 15; more forces a full drain).
      bf16x8_t kf[NDK], vf[NVF], pf[NQB][2];
      auto read_step = [&](int k) {
        kf[k] = kfrag(kslot(IR1()), k);
        if constexpr (PV) vf[k] = vfrag_of(k, vslot(IR2()));
      };
#pragma unroll
      for (int k = 0; k < kAhead; ++k) read_step(k);
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) sn[qb] = zero16();
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int dk = 0; dk < NDK; ++dk) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) sn[qb] = mfma32(kf[dk], qf[qb][dk], sn[qb]);
        if constexpr (PV) pv_step(dk, vf[dk], pfp);
        if (dk + kAhead < NDK) read_step(dk + kAhead);
        softmax_step(dk, sc, pf);
        __builtin_amdgcn_sched_barrier(0);
      }
      softmax_commit(sc, pf);  // after PV(u-1), which used the old max
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        pfp[qb][0] = pf[qb][0];
        pfp[qb][1] = pf[qb][1];
      }
      if (!plan_full(e1)) mask(sn, e1, row0(e1, u + 1), dslot(IR1()));
      // The DMA just issued may stay in flight; everything older (the previous
      // body's DMA, this body's entry load and document DMA) must land.
      wait_vmcnt<2 * NDMA>();
      block_sync_nofence();
      ew[0] = ew[1];
      ew[1] = ew[2];
      ew[2] = ew[3];
      ew[3] = e4;
    };
    using NoPV = std::false_type;
    using WithPV = std::true_type;
    // S(u) lives in sc for even u and in sx for odd u: the bodies alternate
    // the two register sets instead of copying S(u+1) into S(u), so the loop
    // is unrolled over lcm(2, 3) = 6 sub-tiles.
    f32x16_t sx[NQB];
    body(I0(), NoPV(), 0, sc, sx);
    int u = 1;
    for (; u + 6 < U; u += 6) {
      body(I1(), WithPV(), u, sx, sc);
      body(I2(), WithPV(), u + 1, sc, sx);
      body(I0(), WithPV(), u + 2, sx, sc);
      body(I1(), WithPV(), u + 3, sc, sx);
      body(I2(), WithPV(), u + 4, sx, sc);
      body(I0(), WithPV(), u + 5, sc, sx);
    }
    // At most five bodies remain; u % 6 == 1 here.
    if (u + 1 < U) {
      body(I1(), WithPV(), u, sx, sc);
      ++u;
      if (u + 1 < U) {
        body(I2(), WithPV(), u, sc, sx);
        ++u;
        if (u + 1 < U) {
          body(I0(), WithPV(), u, sx, sc);
          ++u;
          if (u + 1 < U) {
            body(I1(), WithPV(), u, sc, sx);
            ++u;
            if (u + 1 < U) {
              body(I2(), WithPV(), u, sx, sc);
              ++u;
            }
          }
        }
      }
    }
    if (u & 1) {
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) sc[qb] = sx[qb];
    }
    // V(u) of the last sub-tile u = U-1 was issued by the last body: every
    // wave's share must land before any wave reads it.
    wait_vmcnt<0>();
    __syncthreads();
    auto vslot_rt = [&](int r) -> const char * { return r == 0 ? vs0 : r == 1 ? vs1 : vs2; };
    const char *vprev = vslot_rt((u + 2) % 3), *vlast = vslot_rt(u % 3);
    bf16x8_t vf[NVF], pf[NQB][2];
#pragma unroll
    for (int f = 0; f < NVF; ++f) vf[f] = vfrag_of(f, vprev);
#pragma unroll
    for (int step = 0; step < NDK; ++step) {
      pv_step(step, vf[step], pfp);
      softmax_step(step, sc, pf);
    }
    softmax_commit(sc, pf);
#pragma unroll
    for (int f = 0; f < NVF; ++f) pv_step(f, vfrag_of(f, vlast), pf);
  }

#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    const float lsum = xor32_sum(l_run[qb]);
    const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
    if (!qv[qb]) continue;
    if (part) {
      // One chunk's normalised output and log-sum-exp, fp32.
      const int64_t prow = (((int64_t)split * a.B + b) * a.Hq + h) * S + qi[qb];
      float *po = a.part_o + prow * DP;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
          typedef float f32x4_t __attribute__((ext_vector_type(4)));
          f32x4_t o4;
#pragma unroll
          for (int x = 0; x < 4; ++x) o4[x] = oacc[qb][db][4 * jq + x] * inv;
          *reinterpret_cast<f32x4_t *>(po + 32 * db + 8 * jq + 4 * hh) = o4;
        }
      if (hh == 0) a.part_lse[prow] = lsum > 0.f ? m_run[qb] + fast_log2(lsum) : -INFINITY;
      continue;
    }
    bf16_t *orow = a.o + b * a.o_sb + (int64_t)qi[qb] * a.o_ss + h * a.o_sh;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) {
        typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
        bf16x4_t o4;
#pragma unroll
        for (int x = 0; x < 4; ++x) o4[x] = (bf16_t)(oacc[qb][db][4 * jq + x] * inv);
        *reinterpret_cast<bf16x4_t *>(orow + 32 * db + 8 * jq + 4 * hh) = o4;
      }
    if (hh == 0)
      a.lse[((int64_t)b * a.Hq + h) * S + qi[qb]] =
          lsum > 0.f ? m_run[qb] + fast_log2(lsum) : -INFINITY;
  }
}

// Merge of the per-chunk outputs of split query tiles: DP/4 threads per
// (pack, head, query row), four output elements each; rows of unsplit tiles
// were written by the attention kernel and are skipped.  Pass 1 takes the
// largest chunk log-sum-exp, pass 2 accumulates the 2^(lse_c - max)-weighted
// chunk outputs with independent (unrolled) 16-byte loads.
template <int DP>
__global__ __launch_bounds__(256) void attn_fwd_combine(FwdArgs a) {
  constexpr int TPR = DP / 4, RPB = 256 / TPR;
  typedef float f32x4_t __attribute__((ext_vector_type(4)));
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  const int d0 = (threadIdx.x % TPR) * 4;
  const int64_t rows = (int64_t)a.B * a.Hq * a.S;
  if (row >= rows) return;
  const int q = (int)(row % a.S);
  const int64_t bh = row / a.S;
  const int h = (int)(bh % a.Hq), b = (int)(bh / a.Hq);
  const int cnt = a.cnt[b * a.nqt + q / a.bm];
  const int nch = (cnt + a.chunk - 1) / a.chunk;
  if (nch <= 1) return;
  const float *pl = a.part_lse + row;
  const float *po = a.part_o + row * DP + d0;
  float mx = -INFINITY;
#pragma unroll 4
  for (int c = 0; c < nch; ++c) mx = fmaxf(mx, pl[c * rows]);
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  float den = 0.f;
  if (mx != -INFINITY) {
#pragma unroll 4
    for (int c = 0; c < nch; ++c) {
      const float w = fast_exp2(pl[c * rows] - mx);
      const f32x4_t o = *reinterpret_cast<const f32x4_t *>(po + c * rows * DP);
      den += w;
      acc += w * o;
    }
  }
  const float inv = den > 0.f ? 1.0f / den : 0.f;
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  bf16x4_t o4;
#pragma unroll
  for (int x = 0; x < 4; ++x) o4[x] = (bf16_t)(acc[x] * inv);
  *reinterpret_cast<bf16x4_t *>(a.o + b * a.o_sb + (int64_t)q * a.o_ss + h * a.o_sh + d0) = o4;
  if (d0 == 0) a.lse[row] = den > 0.f ? mx + fast_log2(den) : -INFINITY;
}

}  // namespace attn
}  // namespace pb

using pb::bf16_t;

extern "C" int pb_attn_fwd(const pb_bhsd *q, const pb_bhsd *k, const pb_bhsd *v,
                           const pb_bhsd *out, float *lse, void *workspace, const int64_t *doc_ids,
                           int64_t doc_stride, const int32_t *plan_counts,
                           const int32_t *plan_lists, int64_t b, int64_t hq, int64_t hkv,
                           int64_t s, int64_t d, float scale, int dtype, void *stream) {
  using namespace pb;
  using namespace pb::attn;
  clear_error();
  int rc = check_attn_shape("pb_attn_fwd", b, hq, hkv, s, d, dtype);
  if (rc) return rc;
  PB_CHECK_ARG(q && k && v && out && lse && doc_ids && plan_counts && plan_lists,
               "pb_attn_fwd: null argument");
  PB_CHECK_ARG(scale > 0.f, "pb_attn_fwd: softmax scale must be positive");
  FwdArgs a;
  a.q = static_cast<const bf16_t *>(q->data);
  a.q_sb = q->stride_b; a.q_sh = q->stride_h; a.q_ss = q->stride_s;
  a.k = static_cast<const bf16_t *>(k->data);
  a.k_sb = k->stride_b; a.k_sh = k->stride_h; a.k_ss = k->stride_s;
  a.v = static_cast<const bf16_t *>(v->data);
  a.v_sb = v->stride_b; a.v_sh = v->stride_h; a.v_ss = v->stride_s;
  a.o = static_cast<bf16_t *>(out->data);
  a.o_sb = out->stride_b; a.o_sh = out->stride_h; a.o_ss = out->stride_s;
  a.lse = lse;
  a.doc = doc_ids;
  a.doc_sb = doc_stride;
  a.cnt = plan_counts;
  a.list = plan_lists;
  a.B = (int)b; a.Hq = (int)hq; a.Hkv = (int)hkv; a.S = (int)s; a.D = (int)d;
  const AttnConfig cfg = attn_config(b, hq, hkv, s, d);
  a.nqt = (int)((s + cfg.fwd_q_tile() - 1) / cfg.fwd_q_tile());
  a.nkt = (int)((s + kKvStep - 1) / kKvStep);
  a.sl2 = scale * kLog2e;
  a.vec = views_vectorizable(d, {q, k, v, out});
  a.chunk = 0;
  a.bm = cfg.fwd_q_tile();
  a.part_o = nullptr;
  a.part_lse = nullptr;
  dim3 grid((unsigned)(a.nqt * b * hq));
  hipStream_t st = as_stream(stream);
  // DMA offsets are 32-bit: one (pack, KV head) view of K / V (S rows) and
  // the pack's document ids must span < 2 GiB.
  const bool pipe = a.vec && (d == 64 || d == 128) && s % 64 == 0 &&
                    (reinterpret_cast<uintptr_t>(doc_ids) & 15) == 0 && doc_stride % 2 == 0 &&
                    s * std::max(k->stride_s, v->stride_s) * 2 < (1LL << 31) &&
                    s * 8 < (1LL << 31);
  if (pipe && cfg.fwd_chunk > 0) {
    PB_CHECK_ARG(workspace != nullptr, "pb_attn_fwd: workspace is required for this shape");
    a.chunk = cfg.fwd_chunk;
    const int64_t prow = (int64_t)cfg.fwd_splits * b * hq * s;
    a.part_o = static_cast<float *>(workspace);
    a.part_lse = reinterpret_cast<float *>(static_cast<char *>(workspace) +
                                           (prow * d * 4 + 255) / 256 * 256);
    grid.x *= (unsigned)cfg.fwd_splits;
  }
  if (pipe) {
#define PB_PIPE(DP, W) hipLaunchKernelGGL((attn_fwd_pipe<DP, 32, W>), grid, dim3(64 * W), 0, st, a)
    if (cfg.fwd_waves == 4) {
      if (d == 128) PB_PIPE(128, 4); else PB_PIPE(64, 4);
    } else {
      if (d == 128) PB_PIPE(128, 2); else PB_PIPE(64, 2);
    }
#undef PB_PIPE
    if (a.chunk > 0) {
      rc = launch_status("pb_attn_fwd");
      if (rc) return rc;
      const int64_t rows = b * hq * s, rpb = 256 / (d / 4);
      const dim3 cgrid((unsigned)((rows + rpb - 1) / rpb));
      if (d == 128) hipLaunchKernelGGL(attn_fwd_combine<128>, cgrid, dim3(256), 0, st, a);
      else hipLaunchKernelGGL(attn_fwd_combine<64>, cgrid, dim3(256), 0, st, a);
    }
  } else {
    // Generic kernel: 32 query rows per wave, same query tile as the plan.
    const int w = cfg.fwd_q_tile() / 32;
#define PB_FWD(DP, W) hipLaunchKernelGGL((attn_fwd_generic<DP, W>), grid, dim3(64 * W), 0, st, a)
    if (w == 4) {
      if (d <= 32) PB_FWD(32, 4); else if (d <= 64) PB_FWD(64, 4); else PB_FWD(128, 4);
    } else {
      if (d <= 32) PB_FWD(32, 2); else if (d <= 64) PB_FWD(64, 2); else PB_FWD(128, 2);
    }
#undef PB_FWD
  }
  return launch_status("pb_attn_fwd");
}
