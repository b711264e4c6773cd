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
//
// Per KV tile a wave computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16, so a
// lane owns one query column: the online-softmax max/sum are lane-local plus
// one exchange with lane^32, and the O^T accumulator of a lane belongs to a
// single query (one rescale factor per lane).  P^T leaves the accumulators as
// the B operand of O^T += V^T P^T directly (see attn_common.hpp for the k-slot
// permutation), so P never touches LDS.  K and V are staged row-major in LDS;
// V^T fragments come from the transposing LDS load ds_read_b64_tr_b16.  The
// next tile's K/V are prefetched into registers while the current one is
// computed.
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
};

template <int DP, int WAVES>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_fwd_kernel(FwdArgs a) {
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

}  // namespace attn
}  // namespace pb

using pb::bf16_t;

extern "C" int pb_attn_fwd(const pb_bhsd *q, const pb_bhsd *k, const pb_bhsd *v,
                           const pb_bhsd *out, float *lse, const int64_t *doc_ids,
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
  dim3 grid((unsigned)(a.nqt * b * hq));
  hipStream_t st = as_stream(stream);
#define PB_FWD(DP, W) hipLaunchKernelGGL((attn_fwd_kernel<DP, W>), grid, dim3(64 * W), 0, st, a)
  if (cfg.fwd_waves == 4) {
    if (d <= 32) PB_FWD(32, 4); else if (d <= 64) PB_FWD(64, 4); else PB_FWD(128, 4);
  } else {
    if (d <= 32) PB_FWD(32, 2); else if (d <= 64) PB_FWD(64, 2); else PB_FWD(128, 2);
  }
#undef PB_FWD
  return launch_status("pb_attn_fwd");
}
