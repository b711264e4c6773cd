// Row-wise cross-entropy over a materialised logits block, for gfx950.
//
// Reference semantics: packbalance/kernels/fused_ce.py:31-89 (_ce_kernel):
//   lse       = max + log(sum exp(x - max))
//   loss      = lse - x[t] + z*lse^2            (0 if t == ignore_index)
//   dlogits   = p*(1 + 2z*lse) - [c == t]       (0 row if t == ignore_index)
// One workgroup per row.  When the row fits in registers (contiguous, at
// most 8 16-byte vectors per thread of a 256- or 1024-thread workgroup: 16K
// / 64K bf16 logits, 8K / 32K fp32) it is read from HBM once and dlogits is
// produced from the registers, so the kernel moves exactly read(logits) +
// write(dlogits); otherwise a streaming two-pass variant with an online
// (max, sum) merge handles any length and strides.  dlogits may have its own
// dtype and strides (``pb_ce_rows_dl``): fp32 logits from a GEMM with fp32
// output give bf16 dlogits for the gradient GEMMs in one pass.
#include <math.h>

#include "common.hpp"

namespace pb {
namespace {

constexpr int kThreads = 256;      // streaming kernel, short register rows
constexpr int kWideThreads = 1024; // register rows beyond 256 threads' reach

template <int kWaves>
__device__ __forceinline__ float block_max(float v, float *red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int k = 1; k < kWaves; ++k) r = fmaxf(r, red[k]);
  return r;
}

template <int kWaves>
__device__ __forceinline__ float block_sum(float v, float *red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int k = 1; k < kWaves; ++k) r += red[k];
  return r;
}

// Merge two (max, sum-of-exp2) pairs in the log2 domain.
__device__ __forceinline__ void merge_ms(float &m, float &s, float m2, float s2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  s = s * fast_exp2(m - mn) + s2 * fast_exp2(m2 - mn);
  m = mn;
}

struct RowOut {
  float lse;     // natural-log logsumexp
  float inv_s;   // 1 / sum exp2(x*log2e - m2)
  float m2;      // max * log2e
};

__device__ __forceinline__ void finish_row(int64_t row, float m2, float s, float tlogit, bool valid,
                                           bool bad_target, float z, float *loss, float *lse_out,
                                           RowOut &o) {
  o.m2 = m2;
  o.inv_s = 1.0f / s;
  o.lse = (m2 + log2f(s)) * kLn2;
  if (threadIdx.x == 0) {
    float l = o.lse - tlogit + z * o.lse * o.lse;
    if (!valid) l = 0.f;
    if (bad_target) l = NAN;
    loss[row] = l;
    if (lse_out) lse_out[row] = o.lse;
  }
}

// VEC dlogits of type U (8, 16 or 32 bytes, aligned to their size) in
// non-temporal 8- or 16-byte stores.
template <typename U, int VEC>
__device__ __forceinline__ void store_vec_nt(U *p, const float (&g)[VEC]) {
  constexpr int B = VEC * (int)sizeof(U);
  if constexpr (B % 16 == 0) {
    constexpr int PER = 16 / sizeof(U);
#pragma unroll
    for (int k = 0; k < B / 16; ++k) {
      u32x4 raw;
      U *e = reinterpret_cast<U *>(&raw);
#pragma unroll
      for (int i = 0; i < PER; ++i) e[i] = from_f32<U>(g[k * PER + i]);
      __builtin_nontemporal_store(raw, reinterpret_cast<u32x4 *>(p) + k);
    }
  } else {
    static_assert(B == 8, "dlogits vector of 8, 16 or 32 bytes");
    u32x2 raw;
    U *e = reinterpret_cast<U *>(&raw);
#pragma unroll
    for (int i = 0; i < VEC; ++i) e[i] = from_f32<U>(g[i]);
    __builtin_nontemporal_store(raw, reinterpret_cast<u32x2 *>(p));
  }
}

template <typename T, typename U, int NV, int THREADS>
__global__ __launch_bounds__(THREADS) void ce_rows_reg(const T *__restrict__ logits, int64_t sm,
                                                       const int64_t *__restrict__ targets,
                                                       float *__restrict__ loss,
                                                       float *__restrict__ lse_out,
                                                       U *__restrict__ dlogits, int64_t dsm, int v,
                                                       int64_t ignore_index, float z) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int kWaves = THREADS / 64;
  __shared__ float red[kWaves];
  const int64_t row = blockIdx.x;
  const T *xr = logits + row * sm;
  const int64_t t = targets[row];
  const bool valid = t != ignore_index;
  const bool bad = valid && (t < 0 || t >= v);
  float x[NV][VEC];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * THREADS + threadIdx.x) * VEC;
    if (c < v) {
      load16_nt<T>(xr + c, x[i]);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        x[i][e] *= kLog2e;
        m = fmaxf(m, x[i][e]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) x[i][e] = -INFINITY;
    }
  }
  m = block_max<kWaves>(m, red);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < VEC; ++e) s += fast_exp2(x[i][e] - m);
  s = block_sum<kWaves>(s, red);
  const float tl = (valid && !bad) ? to_f32(xr[t]) : 0.f;
  RowOut o;
  finish_row(row, m, s, tl, valid, bad, z, loss, lse_out, o);
  if (dlogits == nullptr) return;
  U *dr = dlogits + row * dsm;
  const float scale = valid ? o.inv_s * (1.0f + 2.0f * z * o.lse) : 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * THREADS + threadIdx.x) * VEC;
    if (c < v) {
      float g[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        g[e] = fast_exp2(x[i][e] - m) * scale;
        if (valid && c + e == t) g[e] -= 1.0f;
      }
      store_vec_nt<U, VEC>(dr + c, g);
    }
  }
}

template <typename T, typename U>
__global__ __launch_bounds__(kThreads) void ce_rows_stream(const T *__restrict__ logits, int64_t sm,
                                                           int64_t sv,
                                                           const int64_t *__restrict__ targets,
                                                           float *__restrict__ loss,
                                                           float *__restrict__ lse_out,
                                                           U *__restrict__ dlogits, int64_t dsm,
                                                           int64_t dsv, int64_t v,
                                                           int64_t ignore_index, float z) {
  constexpr int kWaves = kThreads / 64;
  __shared__ float red_m[kWaves], red_s[kWaves];
  const int64_t row = blockIdx.x;
  const T *xr = logits + row * sm;
  const int64_t t = targets[row];
  const bool valid = t != ignore_index;
  const bool bad = valid && (t < 0 || t >= v);
  float m = -INFINITY, s = 0.f;
  for (int64_t c = threadIdx.x; c < v; c += kThreads) {
    const float x = to_f32(xr[c * sv]) * kLog2e;
    if (x > m) {
      s = s * fast_exp2(m - x) + 1.0f;
      m = x;
    } else {
      s += fast_exp2(x - m);
    }
  }
  // Wave merge then block merge of (m, s).
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float m2 = __shfl_xor(m, o), s2 = __shfl_xor(s, o);
    merge_ms(m, s, m2, s2);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    red_m[wave] = m;
    red_s[wave] = s;
  }
  __syncthreads();
  m = red_m[0];
  s = red_s[0];
#pragma unroll
  for (int k = 1; k < kWaves; ++k) merge_ms(m, s, red_m[k], red_s[k]);
  const float tl = (valid && !bad) ? to_f32(xr[t * sv]) : 0.f;
  RowOut o;
  finish_row(row, m, s, tl, valid, bad, z, loss, lse_out, o);
  if (dlogits == nullptr) return;
  U *dr = dlogits + row * dsm;
  const float scale = valid ? o.inv_s * (1.0f + 2.0f * z * o.lse) : 0.f;
  for (int64_t c = threadIdx.x; c < v; c += kThreads) {
    float g = fast_exp2(to_f32(xr[c * sv]) * kLog2e - m) * scale;
    if (valid && c == t) g -= 1.0f;
    dr[c * dsv] = from_f32<U>(g);
  }
}

// Vectors per thread of a register row: 1, 2, 4 or 8, 0 when it does not fit.
inline int reg_vectors(int64_t v, int threads, int vec) {
  const int64_t need = (v + (int64_t)threads * vec - 1) / ((int64_t)threads * vec);
  return need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : need <= 8 ? 8 : 0;
}

template <typename T, typename U>
int run(const void *logits, int64_t sm, int64_t sv, const int64_t *targets, float *loss,
        float *lse, void *dlogits, int64_t dsm, int64_t dsv, int64_t m, int64_t v, int64_t ignore,
        float z, hipStream_t st) {
  constexpr int VEC = 16 / sizeof(T);
  const T *L = static_cast<const T *>(logits);
  U *D = static_cast<U *>(dlogits);
  int nv = 0, threads = kThreads;
  const bool contiguous_rows =
      sv == 1 && (v % VEC) == 0 && (reinterpret_cast<uintptr_t>(logits) % 16) == 0 &&
      ((sm * (int64_t)sizeof(T)) % 16) == 0 &&
      (D == nullptr || (dsv == 1 && (reinterpret_cast<uintptr_t>(dlogits) % 16) == 0 &&
                        ((dsm * (int64_t)sizeof(U)) % 16) == 0));
  if (contiguous_rows) {
    nv = reg_vectors(v, kThreads, VEC);
    if (nv == 0) {
      threads = kWideThreads;
      nv = reg_vectors(v, kWideThreads, VEC);
    }
  }
  dim3 grid((unsigned)m);
#define PB_CE(NV, TH)                                                                         \
  if (nv == NV && threads == TH)                                                              \
    hipLaunchKernelGGL((ce_rows_reg<T, U, NV, TH>), grid, dim3(TH), 0, st, L, sm, targets, loss, \
                       lse, D, dsm, (int)v, ignore, z);                                       \
  else
  PB_CE(1, kThreads) PB_CE(2, kThreads) PB_CE(4, kThreads) PB_CE(8, kThreads)
  PB_CE(4, kWideThreads) PB_CE(8, kWideThreads)
#undef PB_CE
  hipLaunchKernelGGL((ce_rows_stream<T, U>), grid, dim3(kThreads), 0, st, L, sm, sv, targets,
                     loss, lse, D, dsm, dsv, v, ignore, z);
  return launch_status("pb_ce_rows");
}

template <typename T>
int run_dl(int dl_dtype, const void *logits, int64_t sm, int64_t sv, const int64_t *targets,
           float *loss, float *lse, void *dlogits, int64_t dsm, int64_t dsv, int64_t m, int64_t v,
           int64_t ignore, float z, hipStream_t st) {
  switch (dl_dtype) {
    case PB_F32: return run<T, float>(logits, sm, sv, targets, loss, lse, dlogits, dsm, dsv, m, v, ignore, z, st);
    case PB_BF16: return run<T, bf16_t>(logits, sm, sv, targets, loss, lse, dlogits, dsm, dsv, m, v, ignore, z, st);
    default: return run<T, f16_t>(logits, sm, sv, targets, loss, lse, dlogits, dsm, dsv, m, v, ignore, z, st);
  }
}

}  // namespace
}  // namespace pb

extern "C" int pb_ce_rows_dl(const void *logits, int64_t stride_m, int64_t stride_v, int dtype,
                             const int64_t *targets, float *loss, float *lse_out, void *dlogits,
                             int64_t dl_stride_m, int64_t dl_stride_v, int dl_dtype, int64_t m,
                             int64_t v, int64_t ignore_index, float z_loss_coeff, void *stream) {
  using namespace pb;
  clear_error();
  PB_CHECK_ARG(valid_dtype(dtype), "pb_ce_rows: bad dtype %d", dtype);
  PB_CHECK_ARG(valid_dtype(dl_dtype), "pb_ce_rows: bad dlogits dtype %d", dl_dtype);
  PB_CHECK_ARG(m >= 0 && v > 0, "pb_ce_rows: bad shape m=%lld v=%lld", (long long)m, (long long)v);
  PB_CHECK_SUPPORTED(m <= 0x7fffffffLL && v <= 0x7fffffffLL, "pb_ce_rows: too many rows or columns");
  if (m == 0) return PB_OK;
  PB_CHECK_ARG(logits && targets && loss, "pb_ce_rows: null argument");
  hipStream_t st = as_stream(stream);
  switch (dtype) {
    case PB_F32: return run_dl<float>(dl_dtype, logits, stride_m, stride_v, targets, loss, lse_out, dlogits, dl_stride_m, dl_stride_v, m, v, ignore_index, z_loss_coeff, st);
    case PB_BF16: return run_dl<bf16_t>(dl_dtype, logits, stride_m, stride_v, targets, loss, lse_out, dlogits, dl_stride_m, dl_stride_v, m, v, ignore_index, z_loss_coeff, st);
    default: return run_dl<f16_t>(dl_dtype, logits, stride_m, stride_v, targets, loss, lse_out, dlogits, dl_stride_m, dl_stride_v, m, v, ignore_index, z_loss_coeff, st);
  }
}

extern "C" int pb_ce_rows(const void *logits, int64_t stride_m, int64_t stride_v, int dtype,
                          const int64_t *targets, float *loss, float *lse_out, void *dlogits,
                          int64_t m, int64_t v, int64_t ignore_index, float z_loss_coeff,
                          void *stream) {
  return pb_ce_rows_dl(logits, stride_m, stride_v, dtype, targets, loss, lse_out, dlogits,
                       stride_m, stride_v, dtype, m, v, ignore_index, z_loss_coeff, stream);
}
