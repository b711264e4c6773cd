// Fused residual add + RMSNorm for gfx950, with per-operand dtypes.
//
// Reference semantics: the decoder layer's residual stream
// (packbalance/model/llama.py:122-125, `hidden = hidden + sublayer(norm(hidden))`)
// followed by the next RMSNorm (packbalance/kernels/rmsnorm.py:29-72):
//   h = x + delta                       (the new residual, kept in x's dtype)
//   y = h * rstd * w, rstd = 1/sqrt(mean(h^2) + eps)   (y in its own dtype)
// Backward, given dy (for y) and dres (for h, from the rest of the residual
// stream):
//   d = rstd * (dy*w - h_hat * mean(dy*w*h_hat)) + dres,  h_hat = h * rstd
//   dx = d (x's dtype),  ddelta = d (delta's dtype),  dw = sum_rows dy * h_hat
// Fusing the add, the norm and the casts removes the separate fp32 add, the
// per-consumer bf16 casts of y and their backward copies that autocast puts
// around a plain RMSNorm.
//
// Layout: one wave per row, 8 elements per lane and vector (a 16-byte load for
// 16-bit dtypes, two for fp32), rows of up to 2048 elements held in
// registers; longer or misaligned rows take a two-pass loop kernel.  The
// backward writes per-workgroup dw partials summed by a small kernel.  The
// forward streams with non-temporal loads and stores, the backward with
// cached ones (at [4096, 768] rows of the model: backward 15.7 -> 14.9 us
// cached, forward 10.5 -> 10.9 us, so each keeps its faster form).
#include <algorithm>
#include <initializer_list>
#include <utility>

#include "common.hpp"

namespace pb {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

struct AddNormFwd {
  const char *x, *delta, *w;
  char *h, *y;
  float *rstd;
  int64_t xs, ds, hs, ys;  // row strides (elements)
  int xdt, ddt, wdt, ydt;
  int64_t rows;
  int n;
  float eps;
};

struct AddNormBwd {
  const char *dy, *h, *w, *dres;
  const float *rstd;
  char *dx, *ddelta;
  float *partial;
  int64_t dys, hs, drs, dxs, dds;
  int dydt, hdt, wdt, dddt;
  int64_t rows;
  int n, rows_per_wg;
};

__device__ __forceinline__ int esize(int dt) { return dt == PB_F32 ? 4 : 2; }

// 8 consecutive elements of dtype dt at p (16-byte aligned) -> fp32.
__device__ __forceinline__ void ld8(const char *p, int dt, float (&o)[8], bool nt) {
  if (dt == PB_F32) {
    const u32x4 *q = reinterpret_cast<const u32x4 *>(p);
    const u32x4 a = nt ? __builtin_nontemporal_load(q) : q[0];
    const u32x4 b = nt ? __builtin_nontemporal_load(q + 1) : q[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[i] = __uint_as_float(a[i]);
      o[4 + i] = __uint_as_float(b[i]);
    }
  } else {
    const u32x4 *q = reinterpret_cast<const u32x4 *>(p);
    const u32x4 r = nt ? __builtin_nontemporal_load(q) : q[0];
    if (dt == PB_BF16) {
      const bf16_t *e = reinterpret_cast<const bf16_t *>(&r);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = to_f32(e[i]);
    } else {
      const f16_t *e = reinterpret_cast<const f16_t *>(&r);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = to_f32(e[i]);
    }
  }
}

__device__ __forceinline__ void st8(char *p, int dt, const float (&v)[8], bool nt) {
  u32x4 *q = reinterpret_cast<u32x4 *>(p);
  if (dt == PB_F32) {
    u32x4 a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = __float_as_uint(v[i]);
      b[i] = __float_as_uint(v[4 + i]);
    }
    if (nt) {
      __builtin_nontemporal_store(a, q);
      __builtin_nontemporal_store(b, q + 1);
    } else {
      q[0] = a;
      q[1] = b;
    }
  } else {
    u32x4 r;
    if (dt == PB_BF16) {
      bf16_t *e = reinterpret_cast<bf16_t *>(&r);
#pragma unroll
      for (int i = 0; i < 8; ++i) e[i] = from_f32<bf16_t>(v[i]);
    } else {
      f16_t *e = reinterpret_cast<f16_t *>(&r);
#pragma unroll
      for (int i = 0; i < 8; ++i) e[i] = from_f32<f16_t>(v[i]);
    }
    if (nt) __builtin_nontemporal_store(r, q);
    else q[0] = r;
  }
}

__device__ __forceinline__ float ld1(const char *p, int dt) {
  if (dt == PB_F32) return *reinterpret_cast<const float *>(p);
  if (dt == PB_BF16) return to_f32(*reinterpret_cast<const bf16_t *>(p));
  return to_f32(*reinterpret_cast<const f16_t *>(p));
}

__device__ __forceinline__ void st1(char *p, int dt, float v) {
  if (dt == PB_F32) *reinterpret_cast<float *>(p) = v;
  else if (dt == PB_BF16) *reinterpret_cast<bf16_t *>(p) = from_f32<bf16_t>(v);
  else *reinterpret_cast<f16_t *>(p) = from_f32<f16_t>(v);
}

// ---------------------------------------------------------------- forward
template <int NV>
__global__ __launch_bounds__(kThreads) void add_rmsnorm_fwd_reg(AddNormFwd a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int xb = esize(a.xdt), db = esize(a.ddt), wb = esize(a.wdt), yb = esize(a.ydt);
  float h[NV][8], wv[NV][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * 64 + lane) * 8;
    if (c < a.n) {
      ld8(a.x + (row * a.xs + c) * xb, a.xdt, h[i], true);
      if (a.delta) {
        float d[8];
        ld8(a.delta + (row * a.ds + c) * db, a.ddt, d, true);
#pragma unroll
        for (int e = 0; e < 8; ++e) h[i][e] += d[e];
      }
      ld8(a.w + (int64_t)c * wb, a.wdt, wv[i], false);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += h[i][e] * h[i][e];
    }
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)a.n + a.eps);
  if (lane == 0) a.rstd[row] = r;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * 64 + lane) * 8;
    if (c < a.n) {
      if (a.h) st8(a.h + (row * a.hs + c) * xb, a.xdt, h[i], true);
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = h[i][e] * r * wv[i][e];
      st8(a.y + (row * a.ys + c) * yb, a.ydt, o, true);
    }
  }
}

// Any n / alignment: the wave walks its row twice with scalar accesses.
__global__ __launch_bounds__(kThreads) void add_rmsnorm_fwd_loop(AddNormFwd a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int xb = esize(a.xdt), db = esize(a.ddt), wb = esize(a.wdt), yb = esize(a.ydt);
  auto hval = [&](int c) {
    float v = ld1(a.x + (row * a.xs + c) * xb, a.xdt);
    if (a.delta) v += ld1(a.delta + (row * a.ds + c) * db, a.ddt);
    return v;
  };
  float ss = 0.f;
  for (int c = lane; c < a.n; c += 64) {
    const float v = hval(c);
    ss += v * v;
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)a.n + a.eps);
  if (lane == 0) a.rstd[row] = r;
  for (int c = lane; c < a.n; c += 64) {
    const float v = hval(c);
    if (a.h) st1(a.h + (row * a.hs + c) * xb, a.xdt, v);
    st1(a.y + (row * a.ys + c) * yb, a.ydt, v * r * ld1(a.w + (int64_t)c * wb, a.wdt));
  }
}

// ---------------------------------------------------------------- backward
template <int NV>
__global__ __launch_bounds__(kThreads) void add_rmsnorm_bwd_reg(AddNormBwd a) {
  __shared__ float red[kWaves - 1][NV * 8 * 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hb = esize(a.hdt), yb = esize(a.dydt), wb = esize(a.wdt), db = esize(a.dddt);
  const float inv_n = 1.0f / (float)a.n;
  float acc[NV][8], wv[NV][8];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * 64 + lane) * 8;
    if (c < a.n) ld8(a.w + (int64_t)c * wb, a.wdt, wv[i], false);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[i][e] = 0.f;
  }
  const int64_t r0 = (int64_t)blockIdx.x * a.rows_per_wg;
  const int64_t r1 = r0 + a.rows_per_wg < a.rows ? r0 + a.rows_per_wg : a.rows;
#pragma unroll 1
  for (int64_t row = r0 + wave; row < r1; row += kWaves) {
    const float r = a.rstd[row];
    float hh[NV][8], g[NV][8], dr[NV][8];
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * 64 + lane) * 8;
      if (c < a.n) {
        float dy[8];
        ld8(a.h + (row * a.hs + c) * hb, a.hdt, hh[i], false);
        ld8(a.dy + (row * a.dys + c) * yb, a.dydt, dy, false);
        // The incoming residual gradient does not depend on the row sum: load
        // it with the rest so the row costs one memory round trip, not two.
        if (a.dres) ld8(a.dres + (row * a.drs + c) * hb, a.hdt, dr[i], false);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          hh[i][e] *= r;
          g[i][e] = dy[e] * wv[i][e];
          dot += g[i][e] * hh[i][e];
          acc[i][e] += dy[e] * hh[i][e];
        }
      }
    }
    dot = wave_sum(dot) * inv_n;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * 64 + lane) * 8;
      if (c < a.n) {
        float d[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) d[e] = r * (g[i][e] - hh[i][e] * dot);
        if (a.dres) {
#pragma unroll
          for (int e = 0; e < 8; ++e) d[e] += dr[i][e];
        }
        st8(a.dx + (row * a.dxs + c) * hb, a.hdt, d, false);
        if (a.ddelta) st8(a.ddelta + (row * a.dds + c) * db, a.dddt, d, false);
      }
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) red[wave - 1][(i * 8 + e) * 64 + lane] = acc[i][e];
  }
  __syncthreads();
  if (wave == 0) {
    float *out = a.partial + (int64_t)blockIdx.x * a.n;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * 64 + lane) * 8;
      if (c < a.n) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float s = acc[i][e];
#pragma unroll
          for (int k = 0; k < kWaves - 1; ++k) s += red[k][(i * 8 + e) * 64 + lane];
          out[c + e] = s;
        }
      }
    }
  }
}

// Any n / alignment: columns strided over the workgroup, rows in sequence,
// the row dot product reduced through LDS; column c's dw partial is private
// to its thread.
__global__ __launch_bounds__(kThreads) void add_rmsnorm_bwd_loop(AddNormBwd a) {
  __shared__ float red[kWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hb = esize(a.hdt), yb = esize(a.dydt), wb = esize(a.wdt), db = esize(a.dddt);
  const float inv_n = 1.0f / (float)a.n;
  const int64_t r0 = (int64_t)blockIdx.x * a.rows_per_wg;
  const int64_t r1 = r0 + a.rows_per_wg < a.rows ? r0 + a.rows_per_wg : a.rows;
  float *out = a.partial + (int64_t)blockIdx.x * a.n;
  for (int c = threadIdx.x; c < a.n; c += kThreads) out[c] = 0.f;
  __syncthreads();
  for (int64_t row = r0; row < r1; ++row) {
    const float r = a.rstd[row];
    float dot = 0.f;
    for (int c = threadIdx.x; c < a.n; c += kThreads)
      dot += ld1(a.dy + (row * a.dys + c) * yb, a.dydt) * ld1(a.w + (int64_t)c * wb, a.wdt) *
             ld1(a.h + (row * a.hs + c) * hb, a.hdt) * r;
    dot = wave_sum(dot);
    if (lane == 0) red[wave] = dot;
    __syncthreads();
    dot = 0.f;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) dot += red[k];
    dot *= inv_n;
    __syncthreads();
    for (int c = threadIdx.x; c < a.n; c += kThreads) {
      const float hh = ld1(a.h + (row * a.hs + c) * hb, a.hdt) * r;
      const float dy = ld1(a.dy + (row * a.dys + c) * yb, a.dydt);
      float d = r * (dy * ld1(a.w + (int64_t)c * wb, a.wdt) - hh * dot);
      if (a.dres) d += ld1(a.dres + (row * a.drs + c) * hb, a.hdt);
      st1(a.dx + (row * a.dxs + c) * hb, a.hdt, d);
      if (a.ddelta) st1(a.ddelta + (row * a.dds + c) * db, a.dddt, d);
      out[c] += dy * hh;
    }
  }
}

// dw[c] = sum_p partial[p, c] in dtype wdt, or dw[c] += that sum (fp32 dw)
// when accumulate is set.  A workgroup of 16 waves owns 64 columns; wave w
// sums partial rows w, w+16, ... with eight independent accumulators (eight
// loads in flight per lane: the table is a few hundred rows and the kernel
// is bound by load latency, not bandwidth), then the 16 wave sums are
// folded in LDS in a fixed order, so the result is deterministic.
constexpr int kRedWaves = 16;
// The column sum of workgroup column block `blk`; valid in wave 0 (returns
// false for the other waves and for columns past n).
__device__ __forceinline__ bool dw_column_sum(const float *__restrict__ partial, int nparts, int n,
                                              int blk, float (&red)[kRedWaves][64], float &t) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int col = blk * 64 + lane;
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (col < n) {
    int p = w;
    for (; p + 7 * kRedWaves < nparts; p += 8 * kRedWaves) {
#pragma unroll
      for (int k = 0; k < 8; ++k) s[k] += partial[(int64_t)(p + k * kRedWaves) * n + col];
    }
    for (; p < nparts; p += kRedWaves) s[0] += partial[(int64_t)p * n + col];
  }
  red[w][lane] = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
  __syncthreads();
  if (w != 0 || col >= n) return false;
  t = 0.f;
#pragma unroll
  for (int g = 0; g < kRedWaves; ++g) t += red[g][lane];
  return true;
}

__global__ __launch_bounds__(64 * kRedWaves) void add_rmsnorm_dw_reduce(
    const float *__restrict__ partial, char *dw, int wdt, int nparts, int n, int accumulate) {
  __shared__ float red[kRedWaves][64];
  float t;
  if (!dw_column_sum(partial, nparts, n, blockIdx.x, red, t)) return;
  const int col = blockIdx.x * 64 + (threadIdx.x & 63);
  if (accumulate)
    reinterpret_cast<float *>(dw)[col] += t;
  else
    st1(dw + (int64_t)col * esize(wdt), wdt, t);
}

// The same reduction for up to kDwBatch problems in one launch (grid.y =
// problem): dw_i[c] += sum_p partial_i[p, c], partial_i = partials + i *
// stride, fp32 dw.  The per-column arithmetic is the kernel's above, so a
// deferred reduction gives the same bits as the immediate one.
constexpr int kDwBatch = 32;
struct DwBatch {
  float *dw[kDwBatch];
};
__global__ __launch_bounds__(64 * kRedWaves) void rmsnorm_dw_reduce_batched(
    const float *__restrict__ partials, int64_t stride, DwBatch dws, int nparts, int n) {
  __shared__ float red[kRedWaves][64];
  float t;
  if (!dw_column_sum(partials + blockIdx.y * stride, nparts, n, blockIdx.x, red, t)) return;
  dws.dw[blockIdx.y][blockIdx.x * 64 + (threadIdx.x & 63)] += t;
}

// dw = 0 (or unchanged when accumulating) for an empty batch.
__global__ __launch_bounds__(256) void add_rmsnorm_dw_zero(char *dw, int wdt, int n) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c < n) st1(dw + (int64_t)c * esize(wdt), wdt, 0.f);
}

int bwd_nwg(int64_t rows, int &rows_per_wg) {
  int64_t rpw = (rows + 511) / 512;
  if (rpw < kWaves) rpw = kWaves;
  rows_per_wg = (int)rpw;
  const int64_t nwg = (rows + rpw - 1) / rpw;
  return (int)(nwg < 1 ? 1 : nwg);
}

// Vectors per lane for a register-resident row (0 = loop kernel): n % 8 == 0,
// every base and row start 16-byte aligned, n <= 2048.
int pick_nv(int64_t n, std::initializer_list<std::pair<const void *, int64_t>> rows_bytes) {
  if (n % 8) return 0;
  for (const auto &pb : rows_bytes)
    if (pb.first && ((reinterpret_cast<uintptr_t>(pb.first) & 15) || (pb.second & 15))) return 0;
  const int64_t need = (n + 511) / 512;
  return need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : 0;
}

}  // namespace
}  // namespace pb

extern "C" int pb_add_rmsnorm_fwd(const void *x, int64_t x_row_stride, int x_dtype,
                                  const void *delta, int64_t delta_row_stride, int delta_dtype,
                                  void *h_out, int64_t h_row_stride, const void *w, int w_dtype,
                                  void *y, int64_t y_row_stride, int y_dtype, float *rstd,
                                  int64_t rows, int64_t n, float eps, void *stream) {
  using namespace pb;
  clear_error();
  PB_CHECK_ARG(valid_dtype(x_dtype) && valid_dtype(w_dtype) && valid_dtype(y_dtype) &&
                   (!delta || valid_dtype(delta_dtype)),
               "pb_add_rmsnorm_fwd: bad dtype");
  PB_CHECK_ARG(rows >= 0 && n > 0, "pb_add_rmsnorm_fwd: bad shape rows=%lld n=%lld",
               (long long)rows, (long long)n);
  PB_CHECK_SUPPORTED(n <= 65536, "RMSNorm feature dimension is too large for this kernel");
  PB_CHECK_ARG(x_row_stride >= n && y_row_stride >= n && (!delta || delta_row_stride >= n) &&
                   (!h_out || h_row_stride >= n),
               "pb_add_rmsnorm_fwd: row stride < n");
  if (rows == 0) return PB_OK;  // empty tensors may carry null pointers
  PB_CHECK_ARG(x && w && y && rstd, "pb_add_rmsnorm_fwd: null argument");
  AddNormFwd a;
  a.x = static_cast<const char *>(x);
  a.delta = static_cast<const char *>(delta);
  a.w = static_cast<const char *>(w);
  a.h = static_cast<char *>(h_out);
  a.y = static_cast<char *>(y);
  a.rstd = rstd;
  a.xs = x_row_stride; a.ds = delta_row_stride; a.hs = h_row_stride; a.ys = y_row_stride;
  a.xdt = x_dtype; a.ddt = delta ? delta_dtype : x_dtype; a.wdt = w_dtype; a.ydt = y_dtype;
  a.rows = rows;
  a.n = (int)n;
  a.eps = eps;
  const int xb = dtype_bytes(x_dtype), yb = dtype_bytes(y_dtype);
  const int nv = pick_nv(n, {{x, x_row_stride * xb},
                             {delta, delta_row_stride * dtype_bytes(a.ddt)},
                             {h_out, h_row_stride * xb},
                             {w, 0},
                             {y, y_row_stride * yb}});
  dim3 grid((unsigned)((rows + kWaves - 1) / kWaves));
  hipStream_t st = as_stream(stream);
  switch (nv) {
    case 1: hipLaunchKernelGGL((add_rmsnorm_fwd_reg<1>), grid, dim3(kThreads), 0, st, a); break;
    case 2: hipLaunchKernelGGL((add_rmsnorm_fwd_reg<2>), grid, dim3(kThreads), 0, st, a); break;
    case 4: hipLaunchKernelGGL((add_rmsnorm_fwd_reg<4>), grid, dim3(kThreads), 0, st, a); break;
    default: hipLaunchKernelGGL(add_rmsnorm_fwd_loop, grid, dim3(kThreads), 0, st, a);
  }
  return launch_status("pb_add_rmsnorm_fwd");
}

extern "C" int64_t pb_add_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t n) {
  if (rows <= 0 || n <= 0) return 0;
  int rpw;
  return (int64_t)pb::bwd_nwg(rows, rpw) * n * (int64_t)sizeof(float);
}

namespace pb {
namespace {
// The backward kernel alone: dx, ddelta and the dw partials [nwg, n] in
// `workspace` (arguments checked by the caller, rows > 0).  Returns nwg, or
// the (negative) launch status on failure.
int add_rmsnorm_bwd_rows(const void *dy, int64_t dy_row_stride, int dy_dtype, const void *h,
                         int64_t h_row_stride, int h_dtype, const void *w, int w_dtype,
                         const float *rstd, const void *dres, int64_t dres_row_stride, void *dx,
                         int64_t dx_row_stride, void *ddelta, int64_t ddelta_row_stride,
                         int ddelta_dtype, void *workspace, int64_t rows, int64_t n,
                         hipStream_t st, const char *what) {
  AddNormBwd a;
  a.dy = static_cast<const char *>(dy);
  a.h = static_cast<const char *>(h);
  a.w = static_cast<const char *>(w);
  a.dres = static_cast<const char *>(dres);
  a.rstd = rstd;
  a.dx = static_cast<char *>(dx);
  a.ddelta = static_cast<char *>(ddelta);
  a.partial = static_cast<float *>(workspace);
  a.dys = dy_row_stride; a.hs = h_row_stride; a.drs = dres_row_stride;
  a.dxs = dx_row_stride; a.dds = ddelta_row_stride;
  a.dydt = dy_dtype; a.hdt = h_dtype; a.wdt = w_dtype; a.dddt = ddelta ? ddelta_dtype : h_dtype;
  a.rows = rows;
  a.n = (int)n;
  const int nwg = bwd_nwg(rows, a.rows_per_wg);
  const int hb = dtype_bytes(h_dtype);
  const int nv = pick_nv(n, {{dy, dy_row_stride * dtype_bytes(dy_dtype)},
                             {h, h_row_stride * hb},
                             {w, 0},
                             {dres, dres_row_stride * hb},
                             {dx, dx_row_stride * hb},
                             {ddelta, ddelta_row_stride * dtype_bytes(a.dddt)}});
  dim3 grid((unsigned)nwg);
  switch (nv) {
    case 1: hipLaunchKernelGGL((add_rmsnorm_bwd_reg<1>), grid, dim3(kThreads), 0, st, a); break;
    case 2: hipLaunchKernelGGL((add_rmsnorm_bwd_reg<2>), grid, dim3(kThreads), 0, st, a); break;
    case 4: hipLaunchKernelGGL((add_rmsnorm_bwd_reg<4>), grid, dim3(kThreads), 0, st, a); break;
    default: hipLaunchKernelGGL(add_rmsnorm_bwd_loop, grid, dim3(kThreads), 0, st, a);
  }
  const int s = launch_status(what);
  return s < 0 ? s : nwg;
}

int check_bwd_args(const char *what, int dy_dtype, int h_dtype, int w_dtype, const void *ddelta,
                   int ddelta_dtype, int64_t rows, int64_t n, int64_t dy_row_stride,
                   int64_t h_row_stride, int64_t dx_row_stride, const void *dres,
                   int64_t dres_row_stride, int64_t ddelta_row_stride) {
  PB_CHECK_ARG(valid_dtype(dy_dtype) && valid_dtype(h_dtype) && valid_dtype(w_dtype) &&
                   (!ddelta || valid_dtype(ddelta_dtype)),
               "%s: bad dtype", what);
  PB_CHECK_ARG(rows >= 0 && n > 0, "%s: bad shape", what);
  PB_CHECK_SUPPORTED(n <= 65536, "RMSNorm feature dimension is too large for this kernel");
  PB_CHECK_ARG(dy_row_stride >= n && h_row_stride >= n && dx_row_stride >= n &&
                   (!dres || dres_row_stride >= n) && (!ddelta || ddelta_row_stride >= n),
               "%s: row stride < n", what);
  return PB_OK;
}
}  // namespace
}  // namespace pb

extern "C" int pb_add_rmsnorm_bwd(const void *dy, int64_t dy_row_stride, int dy_dtype,
                                  const void *h, int64_t h_row_stride, int h_dtype, const void *w,
                                  int w_dtype, const float *rstd, const void *dres,
                                  int64_t dres_row_stride, void *dx, int64_t dx_row_stride,
                                  void *ddelta, int64_t ddelta_row_stride, int ddelta_dtype,
                                  void *dw, int dw_accumulate, void *workspace, int64_t rows,
                                  int64_t n, void *stream) {
  using namespace pb;
  clear_error();
  int rc = check_bwd_args("pb_add_rmsnorm_bwd", dy_dtype, h_dtype, w_dtype, ddelta, ddelta_dtype,
                          rows, n, dy_row_stride, h_row_stride, dx_row_stride, dres,
                          dres_row_stride, ddelta_row_stride);
  if (rc) return rc;
  PB_CHECK_ARG(w && dw, "pb_add_rmsnorm_bwd: null weight or dw");
  PB_CHECK_ARG(!dw_accumulate || w_dtype == PB_F32,
               "pb_add_rmsnorm_bwd: dw_accumulate needs an fp32 weight (and dw)");
  hipStream_t st = as_stream(stream);
  if (rows == 0) {
    if (!dw_accumulate)
      hipLaunchKernelGGL(add_rmsnorm_dw_zero, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                         static_cast<char *>(dw), w_dtype, (int)n);
    return launch_status("pb_add_rmsnorm_bwd(empty)");
  }
  PB_CHECK_ARG(dy && h && rstd && dx, "pb_add_rmsnorm_bwd: null argument");
  PB_CHECK_ARG(workspace != nullptr, "pb_add_rmsnorm_bwd: workspace is required");
  const int nwg = add_rmsnorm_bwd_rows(dy, dy_row_stride, dy_dtype, h, h_row_stride, h_dtype, w,
                                       w_dtype, rstd, dres, dres_row_stride, dx, dx_row_stride,
                                       ddelta, ddelta_row_stride, ddelta_dtype, workspace, rows, n,
                                       st, "pb_add_rmsnorm_bwd");
  if (nwg < 0) return nwg;
  hipLaunchKernelGGL(add_rmsnorm_dw_reduce, dim3((unsigned)((n + 63) / 64)), dim3(64 * kRedWaves),
                     0, st, static_cast<const float *>(workspace), static_cast<char *>(dw), w_dtype,
                     nwg, (int)n, dw_accumulate ? 1 : 0);
  return launch_status("pb_add_rmsnorm_bwd(dw)");
}

extern "C" int pb_add_rmsnorm_bwd_partials(const void *dy, int64_t dy_row_stride, int dy_dtype,
                                           const void *h, int64_t h_row_stride, int h_dtype,
                                           const void *w, int w_dtype, const float *rstd,
                                           const void *dres, int64_t dres_row_stride, void *dx,
                                           int64_t dx_row_stride, void *ddelta,
                                           int64_t ddelta_row_stride, int ddelta_dtype,
                                           float *partials, int64_t rows, int64_t n,
                                           void *stream) {
  using namespace pb;
  clear_error();
  int rc = check_bwd_args("pb_add_rmsnorm_bwd_partials", dy_dtype, h_dtype, w_dtype, ddelta,
                          ddelta_dtype, rows, n, dy_row_stride, h_row_stride, dx_row_stride, dres,
                          dres_row_stride, ddelta_row_stride);
  if (rc) return rc;
  if (rows == 0) return PB_OK;  // no partial rows: the reduction adds nothing
  PB_CHECK_ARG(dy && h && w && rstd && dx && partials, "pb_add_rmsnorm_bwd_partials: null argument");
  const int nwg = add_rmsnorm_bwd_rows(dy, dy_row_stride, dy_dtype, h, h_row_stride, h_dtype, w,
                                       w_dtype, rstd, dres, dres_row_stride, dx, dx_row_stride,
                                       ddelta, ddelta_row_stride, ddelta_dtype, partials, rows, n,
                                       as_stream(stream), "pb_add_rmsnorm_bwd_partials");
  return nwg < 0 ? nwg : PB_OK;
}

extern "C" int pb_rmsnorm_dw_reduce_batched(const float *partials, int64_t problem_stride,
                                            float *const *dw, int64_t count, int64_t rows,
                                            int64_t n, void *stream) {
  using namespace pb;
  clear_error();
  PB_CHECK_ARG(count >= 0 && rows >= 0 && n > 0 && n <= 65536,
               "pb_rmsnorm_dw_reduce_batched: bad shape count=%lld rows=%lld n=%lld",
               (long long)count, (long long)rows, (long long)n);
  if (count == 0 || rows == 0) return PB_OK;
  int rpw;
  const int nparts = bwd_nwg(rows, rpw);
  PB_CHECK_ARG(partials && dw && problem_stride >= (int64_t)nparts * n,
               "pb_rmsnorm_dw_reduce_batched: null argument or problem stride < partial table");
  hipStream_t st = as_stream(stream);
  for (int64_t i0 = 0; i0 < count; i0 += kDwBatch) {
    const int m = (int)std::min<int64_t>(kDwBatch, count - i0);
    DwBatch b{};
    for (int i = 0; i < m; ++i) {
      PB_CHECK_ARG(dw[i0 + i] != nullptr, "pb_rmsnorm_dw_reduce_batched: null dw[%lld]",
                   (long long)(i0 + i));
      b.dw[i] = dw[i0 + i];
    }
    hipLaunchKernelGGL(rmsnorm_dw_reduce_batched, dim3((unsigned)((n + 63) / 64), (unsigned)m),
                       dim3(64 * kRedWaves), 0, st, partials + i0 * problem_stride, problem_stride,
                       b, nparts, (int)n);
    const int s = launch_status("pb_rmsnorm_dw_reduce_batched");
    if (s) return s;
  }
  return PB_OK;
}
