// Document-masked GQA attention backward for gfx950 (bf16 in, fp32 accumulate).
//
// Reference: the FlexAttention backward of packbalance/model/attention.py:116-122
// (gradients of softmax(scale * Q K^T | doc mask) V, dK/dV summed over each
// GQA group as enable_gqa does).  With P = softmax, D_i = rowsum(dO_i * O_i):
//   dV = P^T dO,  dP = dO V^T,  dS = P * (dP - D),
//   dQ = scale * dS K,  dK = scale * dS^T Q.
//
// Three kernels, no atomics (results are run-to-run deterministic):
//   attn_bwd_delta  D = rowsum(dO * O) per (pack, head, query).
//   attn_bwd_dkdv   one workgroup per (pack, KV head, 128-row KV tile); wave w
//                   owns 32 KV rows.  It walks every query head of its GQA group
//                   and every 32-row query tile the plan lists for the KV tile,
//                   so dK/dV accumulate in registers across the whole group.
//                   S = Q K^T is computed with lane <-> KV row, which lets P^T
//                   and dS^T feed the dV / dK MFMAs straight from the
//                   accumulators; Q and dO are staged in LDS row-major (for S,
//                   dP) and transposed (for dK, dV).
//   attn_bwd_dq     one workgroup per (pack, query head, 128-row query tile),
//                   shaped like the forward: lane <-> query row, recomputes S^T
//                   and dP^T per 64-row KV tile and accumulates dQ^T = K^T dS^T.
#include "attn_common.hpp"

namespace pb {
namespace attn {

constexpr int kKvBN = 128;  // dK/dV kernel: KV rows per workgroup
constexpr int kKvBM = 32;   // dK/dV kernel: query rows per step
constexpr int kDqBM = 128;  // dQ kernel: query rows per workgroup
constexpr int kDqBN = 64;   // dQ kernel: KV rows per step

int attn_bwd_tile(int kernel, int which) {
  if (kernel == 1) return which == 0 ? kKvBM : kKvBN;
  if (kernel == 2) return which == 0 ? kDqBM : kDqBN;
  return -1;
}

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
  int B, Hq, Hkv, S, D;
  int nqt_dq, nkt_dq, nqt_kv, nkt_kv;
  float sl2, scale;
  int vec;
};

// ---------------------------------------------------------------- delta
// One thread per (b, s, h) row, h fastest: neighbouring threads read
// neighbouring rows of the [B, S, H, D] memory the model produces.
__global__ __launch_bounds__(256) void attn_bwd_delta(BwdArgs a) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)a.B * a.S * a.Hq;
  if (t >= total) return;
  const int h = (int)(t % a.Hq);
  const int64_t s = (t / a.Hq) % a.S;
  const int b = (int)(t / ((int64_t)a.Hq * a.S));
  const bf16_t *o = a.o.row(b, h, s);
  const bf16_t *g = a.dout.row(b, h, s);
  float acc = 0.f;
  if (a.vec) {
    for (int d = 0; d < a.D; d += 8) {
      const bf16x8_t x = *reinterpret_cast<const bf16x8_t *>(o + d);
      const bf16x8_t y = *reinterpret_cast<const bf16x8_t *>(g + d);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc += (float)x[i] * (float)y[i];
    }
  } else {
    for (int d = 0; d < a.D; ++d) acc += (float)o[d] * (float)g[d];
  }
  a.delta[((int64_t)b * a.Hq + h) * a.S + s] = acc;
}

// ---------------------------------------------------------------- dK, dV
template <int DP>
__global__ __launch_bounds__(256) void attn_bwd_dkdv(BwdArgs a) {
  constexpr int BN = kKvBN, BM = kKvBM;
  constexpr int QP = DP + 8;  // row-major pitch (elements)
  constexpr int TP = BM + 4;  // transposed pitch (elements)
  constexpr int NDK = DP / 16, NDB = DP / 32, CH = DP / 8;
  constexpr int NCH = BM * CH;  // 16-byte chunks of one [BM x DP] tile
  __shared__ __align__(16) bf16_t Qs[BM * QP];
  __shared__ __align__(16) bf16_t Gs[BM * QP];  // dO, row-major
  __shared__ __align__(16) bf16_t Qt[DP * TP];
  __shared__ __align__(16) bf16_t Gt[DP * TP];  // dO, transposed
  __shared__ float lse_s[BM], dlt_s[BM];
  __shared__ int64_t qdoc_s[BM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hh = lane >> 5, l32 = lane & 31;
  const int nbh = a.B * a.Hkv;
  const int kt = (int)(blockIdx.x / nbh);  // early KV tiles are attended most: first
  const int rem = (int)(blockIdx.x % nbh);
  const int b = rem / a.Hkv, hk = rem - (rem / a.Hkv) * a.Hkv;
  const int G = a.Hq / a.Hkv;
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
  for (int g = 0; g < G; ++g) {
    const int h = hk * G + g;
    const float *lse_row = a.lse + ((int64_t)b * a.Hq + h) * a.S;
    const float *dlt_row = a.delta + ((int64_t)b * a.Hq + h) * a.S;
    for (int it = 0; it < cnt; ++it) {
      const int e = lst[it];
      const int q0 = plan_tile(e) * BM;
      const bool full = plan_full(e);
      __syncthreads();
      for (int c = tid; c < 2 * NCH; c += 256) {
        const int which = c / NCH, cc = c - which * NCH;
        const int row = cc / CH, col = (cc % CH) * 8;
        const int qr = q0 + row;
        const bool ok = qr < a.S;
        const View &src = which ? a.dout : a.q;
        const bf16x8_t x = load_row8(src.row(b, h, ok ? qr : 0), col, a.D, ok, vec);
        bf16_t *rm = which ? Gs : Qs;
        bf16_t *tr = which ? Gt : Qt;
        *reinterpret_cast<bf16x8_t *>(&rm[row * QP + col]) = x;
#pragma unroll
        for (int xi = 0; xi < 8; ++xi) tr[(col + xi) * TP + row] = x[xi];
      }
      if (tid < BM) {
        const int qr = q0 + tid;
        const bool ok = qr < a.S;
        lse_s[tid] = ok ? lse_row[qr] : 0.f;
        dlt_s[tid] = ok ? dlt_row[qr] : 0.f;
        qdoc_s[tid] = ok ? docb[qr] : 0;
      }
      __syncthreads();

      // S = Q K^T and dP = dO V^T for 32 query rows x this wave's 32 KV rows.
      f32x16_t sacc = zero16(), pacc = zero16();
#pragma unroll
      for (int dk = 0; dk < NDK; ++dk) {
        const bf16x8_t qa = *reinterpret_cast<const bf16x8_t *>(&Qs[l32 * QP + 16 * dk + 8 * hh]);
        sacc = mfma32(qa, kf[dk], sacc);
        const bf16x8_t ga = *reinterpret_cast<const bf16x8_t *>(&Gs[l32 * QP + 16 * dk + 8 * hh]);
        pacc = mfma32(ga, vf[dk], pacc);
      }
      bf16x8_t pf[2], dsf[2];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int qr = 8 * (j >> 2) + 4 * hh + (j & 3);
        const int q = q0 + qr;
        const bool ok = full || (q < a.S && kvvalid && q >= kv && qdoc_s[qr] == kvdoc);
        const float p = ok ? fast_exp2(sacc[j] * a.sl2 - lse_s[qr]) : 0.f;
        const float ds = p * (pacc[j] - dlt_s[qr]);
        pf[j >> 3][j & 7] = (bf16_t)p;
        dsf[j >> 3][j & 7] = (bf16_t)ds;
      }
      // dV += P^T dO, dK += dS^T Q; B operands read the transposed tiles.
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int qk = 0; qk < 2; ++qk) {
          const int off = (32 * db + l32) * TP + 16 * qk + 4 * hh;
          const u32x2 g_lo = *reinterpret_cast<const u32x2 *>(&Gt[off]);
          const u32x2 g_hi = *reinterpret_cast<const u32x2 *>(&Gt[off + 8]);
          u32x4 gb = {g_lo[0], g_lo[1], g_hi[0], g_hi[1]};
          dv_acc[db] = mfma32(pf[qk], *reinterpret_cast<bf16x8_t *>(&gb), dv_acc[db]);
          const u32x2 q_lo = *reinterpret_cast<const u32x2 *>(&Qt[off]);
          const u32x2 q_hi = *reinterpret_cast<const u32x2 *>(&Qt[off + 8]);
          u32x4 qb = {q_lo[0], q_lo[1], q_hi[0], q_hi[1]};
          dk_acc[db] = mfma32(dsf[qk], *reinterpret_cast<bf16x8_t *>(&qb), dk_acc[db]);
        }
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
        a.dk.row(b, hk, kvr)[d] = (bf16_t)(dk_acc[db][j] * a.scale);
        a.dv.row(b, hk, kvr)[d] = (bf16_t)dv_acc[db][j];
      }
    }
  }
}

// ---------------------------------------------------------------- dQ
template <int DP>
__global__ __launch_bounds__(256) void attn_bwd_dq(BwdArgs a) {
  constexpr int BM = kDqBM, BN = kDqBN;
  constexpr int KP = DP + 8, VP = BN + 4;
  constexpr int NDK = DP / 16, NDB = DP / 32, CH = DP / 8;
  constexpr int NLD = BN * CH / 256;
  static_assert(NLD >= 1 && BN * CH % 256 == 0, "tile/thread mismatch");
  __shared__ __align__(16) bf16_t Ks[BN * KP];
  __shared__ __align__(16) bf16_t Vs[BN * KP];
  __shared__ __align__(16) bf16_t Kt[DP * VP];
  __shared__ int64_t kdoc[BN];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hh = lane >> 5, l32 = lane & 31;
  const int bh = a.B * a.Hq;
  const int qt = a.nqt_dq - 1 - (int)(blockIdx.x / bh);
  const int rem = (int)(blockIdx.x % bh);
  const int b = rem / a.Hq, h = rem - (rem / a.Hq) * a.Hq;
  const int hk = h / (a.Hq / a.Hkv);
  const bool vec = a.vec != 0;
  const int64_t *docb = a.doc + b * a.doc_sb;

  const int qi = qt * BM + wave * 32 + l32;
  const bool qvalid = qi < a.S;
  const int64_t qdoc = qvalid ? docb[qi] : 0;
  const float lse2 = qvalid ? a.lse[((int64_t)b * a.Hq + h) * a.S + qi] : 0.f;
  const float dlt = qvalid ? a.delta[((int64_t)b * a.Hq + h) * a.S + qi] : 0.f;
  bf16x8_t qf[NDK], gf[NDK];
  {
    const int64_t r = qvalid ? qi : 0;
    const bf16_t *qrow = a.q.row(b, h, r), *grow = a.dout.row(b, h, r);
#pragma unroll
    for (int dk = 0; dk < NDK; ++dk) {
      qf[dk] = load_row8(qrow, 16 * dk + 8 * hh, a.D, qvalid, vec);
      gf[dk] = load_row8(grow, 16 * dk + 8 * hh, a.D, qvalid, vec);
    }
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
      const int c = tid + 256 * i;
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
      const int c = tid + 256 * i;
      const int row = c / CH, col = (c % CH) * 8;
      *reinterpret_cast<bf16x8_t *>(&Ks[row * KP + col]) = kr[i];
      *reinterpret_cast<bf16x8_t *>(&Vs[row * KP + col]) = vr[i];
#pragma unroll
      for (int x = 0; x < 8; ++x) Kt[(col + x) * VP + row] = kr[i][x];
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
        const float p = ok ? fast_exp2(sacc[j] * a.sl2 - lse2) : 0.f;
        dsf[2 * blk + (j >> 3)][j & 7] = (bf16_t)(p * (pacc[j] - dlt));
      }
    }
    // dQ^T += K^T dS^T; A = K^T rows d, k slots kv = 16kk + pi(hh, s).
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const bf16_t *krow = &Kt[(32 * db + l32) * VP + 16 * kk + 4 * hh];
        const u32x2 lo = *reinterpret_cast<const u32x2 *>(krow);
        const u32x2 hi = *reinterpret_cast<const u32x2 *>(krow + 8);
        u32x4 ka = {lo[0], lo[1], hi[0], hi[1]};
        dq_acc[db] = mfma32(*reinterpret_cast<bf16x8_t *>(&ka), dsf[kk], dq_acc[db]);
      }
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

extern "C" int pb_attn_tile(int kernel, int64_t head_dim, int which) {
  (void)head_dim;
  if (kernel == 0) return which == 0 ? pb::attn::kFwdBM : pb::attn::kFwdBN;
  return pb::attn::attn_bwd_tile(kernel, which);
}

extern "C" int pb_attn_bwd(const pb_bhsd *q, const pb_bhsd *k, const pb_bhsd *v,
                           const pb_bhsd *out, const pb_bhsd *dout, const pb_bhsd *dq,
                           const pb_bhsd *dk, const pb_bhsd *dv, const float *lse,
                           float *delta_ws, const int64_t *doc_ids, int64_t doc_stride,
                           const int32_t *q_plan_counts, const int32_t *q_plan_lists,
                           const int32_t *kv_plan_counts, const int32_t *kv_plan_lists,
                           int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t d, float scale,
                           int dtype, void *stream) {
  using namespace pb;
  using namespace pb::attn;
  clear_error();
  int rc = check_attn_shape("pb_attn_bwd", b, hq, hkv, s, d, dtype);
  if (rc) return rc;
  PB_CHECK_ARG(q && k && v && out && dout && dq && dk && dv && lse && delta_ws && doc_ids &&
                   q_plan_counts && q_plan_lists && kv_plan_counts && kv_plan_lists,
               "pb_attn_bwd: null argument");
  BwdArgs a;
  a.q = view_of(q); a.k = view_of(k); a.v = view_of(v); a.o = view_of(out);
  a.dout = view_of(dout); a.dq = view_of(dq); a.dk = view_of(dk); a.dv = view_of(dv);
  a.lse = lse;
  a.delta = delta_ws;
  a.doc = doc_ids;
  a.doc_sb = doc_stride;
  a.qcnt = q_plan_counts; a.qlist = q_plan_lists;
  a.kcnt = kv_plan_counts; a.klist = kv_plan_lists;
  a.B = (int)b; a.Hq = (int)hq; a.Hkv = (int)hkv; a.S = (int)s; a.D = (int)d;
  a.nqt_dq = (int)((s + kDqBM - 1) / kDqBM);
  a.nkt_dq = (int)((s + kDqBN - 1) / kDqBN);
  a.nqt_kv = (int)((s + kKvBM - 1) / kKvBM);
  a.nkt_kv = (int)((s + kKvBN - 1) / kKvBN);
  a.sl2 = scale * kLog2e;
  a.scale = scale;
  a.vec = views_vectorizable(d, {q, k, v, out, dout, dq, dk, dv});
  hipStream_t st = as_stream(stream);
  const int64_t rows = b * hq * s;
  hipLaunchKernelGGL(attn_bwd_delta, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st, a);
  rc = launch_status("pb_attn_bwd(delta)");
  if (rc) return rc;
  dim3 g_kv((unsigned)(a.nkt_kv * b * hkv)), g_q((unsigned)(a.nqt_dq * b * hq));
  if (d <= 32) {
    hipLaunchKernelGGL(attn_bwd_dkdv<32>, g_kv, dim3(256), 0, st, a);
    hipLaunchKernelGGL(attn_bwd_dq<32>, g_q, dim3(256), 0, st, a);
  } else if (d <= 64) {
    hipLaunchKernelGGL(attn_bwd_dkdv<64>, g_kv, dim3(256), 0, st, a);
    hipLaunchKernelGGL(attn_bwd_dq<64>, g_q, dim3(256), 0, st, a);
  } else {
    hipLaunchKernelGGL(attn_bwd_dkdv<128>, g_kv, dim3(256), 0, st, a);
    hipLaunchKernelGGL(attn_bwd_dq<128>, g_q, dim3(256), 0, st, a);
  }
  return launch_status("pb_attn_bwd");
}
