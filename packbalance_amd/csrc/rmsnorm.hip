// RMSNorm forward and backward for gfx950.
//
// Reference semantics: packbalance/kernels/rmsnorm.py:29-72 (Triton kernels)
// and rmsnorm.py:77-119 (_RMSNorm: rstd cached in fp32, dw = sum_r dy*x_hat).
//
// Layout: one 64-lane wavefront owns one row at a time; every lane moves
// 16-byte vectors, so a row of n elements is read as n*sizeof(T)/1024
// fully-coalesced wave loads.  When a row fits in registers (n <= 64*VEC*NV)
// it is read from HBM exactly once; the reduction is a wave64 butterfly, so
// no LDS or block barrier sits on the forward path.  The backward also
// accumulates the per-column dw partial sums of the rows a workgroup owns and
// writes one fp32 partial row per workgroup; a second small kernel sums the
// partials (the reference does this with two extra eager passes over x, dy).
#include <mutex>

#include "common.hpp"

namespace pb {
namespace {

constexpr int kWaves = 4;  // waves per workgroup
constexpr int kThreads = 64 * kWaves;

// Load `N` consecutive elements of T at p (p aligned to N*sizeof(T) bytes up
// to 16) into fp32.
template <typename T, int N>
__device__ __forceinline__ void load_vec(const T *p, float (&o)[N]) {
  constexpr int kBytes = N * sizeof(T);
  static_assert(kBytes % 8 == 0, "vector of at least 8 bytes");
  if constexpr (kBytes >= 16) {
#pragma unroll
    for (int c = 0; c < kBytes / 16; ++c) {
      u32x4 raw = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const char *>(p) + 16 * c);
      const T *e = reinterpret_cast<const T *>(&raw);
#pragma unroll
      for (int i = 0; i < 16 / (int)sizeof(T); ++i) o[c * (16 / sizeof(T)) + i] = to_f32(e[i]);
    }
  } else {
    u32x2 raw = *reinterpret_cast<const u32x2 *>(p);
    const T *e = reinterpret_cast<const T *>(&raw);
#pragma unroll
    for (int i = 0; i < N; ++i) o[i] = to_f32(e[i]);
  }
}

template <typename T, int N>
__device__ __forceinline__ void store_vec(T *p, const float (&v)[N]) {
  static_assert(N * sizeof(T) == 16, "16-byte store");
  u32x4 raw;
  T *e = reinterpret_cast<T *>(&raw);
#pragma unroll
  for (int i = 0; i < N; ++i) e[i] = from_f32<T>(v[i]);
  *reinterpret_cast<u32x4 *>(p) = raw;
}

// ---------------------------------------------------------------- forward
// Register-resident row: NV vectors of VEC elements per lane.  Each wave walks
// rows wave_id, wave_id + total_waves, ... and loads the next row while it
// reduces and writes the current one, so a wave keeps a row of reads in
// flight at all times; w is loaded once per wave and kept packed.
template <typename TX, typename TW, int NV>
__global__ __launch_bounds__(kThreads) void rmsnorm_fwd_reg(
    const TX *__restrict__ x, int64_t xs, const TW *__restrict__ w, TX *__restrict__ y, int64_t ys,
    float *__restrict__ rstd_out, int64_t rows, int n, float eps) {
  constexpr int VEC = 16 / sizeof(TX);
  constexpr int WB = VEC * sizeof(TW);  // bytes of w per vector
  typedef unsigned wraw_t __attribute__((ext_vector_type(WB / 4)));
  const int lane = threadIdx.x & 63;
  const int64_t step = (int64_t)gridDim.x * kWaves;
  int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  wraw_t wraw[NV];
  u32x4 cur[NV];
  auto load_row = [&](int64_t r, u32x4 (&dst)[NV]) {
    const TX *xr = x + r * xs;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * 64 + lane) * VEC;
      if (c < n) dst[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(xr + c));
    }
  };
  load_row(row, cur);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * 64 + lane) * VEC;
    if (c < n) wraw[i] = *reinterpret_cast<const wraw_t *>(w + c);
  }
#pragma unroll 1
  for (; row < rows; row += step) {
    u32x4 nxt[NV];
    if (row + step < rows) load_row(row + step, nxt);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * 64 + lane) * VEC;
      if (c < n) {
        const TX *e = reinterpret_cast<const TX *>(&cur[i]);
#pragma unroll
        for (int k = 0; k < VEC; ++k) ss += to_f32(e[k]) * to_f32(e[k]);
      }
    }
    ss = wave_sum_full(ss);
    const float r = 1.0f / sqrtf(ss / (float)n + eps);
    if (lane == 0) rstd_out[row] = r;
    TX *yr = y + row * ys;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * 64 + lane) * VEC;
      if (c < n) {
        const TX *e = reinterpret_cast<const TX *>(&cur[i]);
        const TW *we = reinterpret_cast<const TW *>(&wraw[i]);
        float o[VEC];
#pragma unroll
        for (int k = 0; k < VEC; ++k) o[k] = to_f32(e[k]) * r * to_f32(we[k]);
        store16_nt<TX>(yr + c, o);
      }
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) cur[i] = nxt[i];
  }
}

// Workgroups of the register-resident forward: enough for four 4-wave
// workgroups per CU (rows walked in a loop beyond that).
inline unsigned fwd_reg_grid(int64_t rows) {
  const int64_t want = (rows + kWaves - 1) / kWaves;
  return (unsigned)(want < 1024 ? want : 1024);
}

// General row (any n, any alignment): two passes over the row, scalar loads.
template <typename TX, typename TW>
__global__ __launch_bounds__(kThreads) void rmsnorm_fwd_loop(
    const TX *__restrict__ x, int64_t xs, const TW *__restrict__ w, TX *__restrict__ y, int64_t ys,
    float *__restrict__ rstd_out, int64_t rows, int n, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const TX *xr = x + row * xs;
  float ss = 0.f;
  for (int c = lane; c < n; c += 64) {
    float t = to_f32(xr[c]);
    ss += t * t;
  }
  ss = wave_sum_full(ss);
  const float r = 1.0f / sqrtf(ss / (float)n + eps);
  if (lane == 0) rstd_out[row] = r;
  TX *yr = y + row * ys;
  for (int c = lane; c < n; c += 64) yr[c] = from_f32<TX>(to_f32(xr[c]) * r * to_f32(w[c]));
}

// ---------------------------------------------------------------- backward
// Rows are walked grid-stride: wave w of workgroup b takes rows b*kWaves + w,
// then every gridDim.x*kWaves-th row, so at any time the whole grid reads one
// compact window of rows (at [32768, 4096] bf16, 5.27 TB/s against 5.0 with a
// contiguous block of rows per workgroup).  Per row a wave streams x and dy once (non-temporal,
// kept as raw 16-byte vectors), forms dot = sum(dy*w*x_hat) and the dw
// partial in one pass over the registers, and dx = r*(dy*w - x_hat*dot) in a
// second; w is loaded once per wave.  The next row is loaded into the same
// registers vector by vector as the current row's dx leaves (no second row of
// registers: 224 in all at bf16 n = 4096, two waves per SIMD).  dw partials
// are reduced across the waves in LDS and written as one fp32 row per
// workgroup.
template <typename TX, typename TW, int NV>
__global__ __launch_bounds__(kThreads) void rmsnorm_bwd_reg(
    const TX *__restrict__ dy, int64_t dys, const TX *__restrict__ x, int64_t xs,
    const TW *__restrict__ w, const float *__restrict__ rstd, TX *__restrict__ dx, int64_t dxs,
    float *__restrict__ partial, int64_t rows, int n) {
  constexpr int VEC = 16 / sizeof(TX);
  __shared__ float red[kWaves - 1][NV * VEC * 64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const float inv_n = 1.0f / (float)n;
  // w stays packed in its own type (VEC elements per lane and vector) and is
  // widened where it is used.
  constexpr int WB = VEC * sizeof(TW);  // bytes of w per vector
  typedef unsigned wraw_t __attribute__((ext_vector_type(WB / 4)));
  float acc[NV][VEC];
  wraw_t wraw[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * 64 + lane) * VEC;
    if (c < n) wraw[i] = *reinterpret_cast<const wraw_t *>(w + c);
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[i][e] = 0.f;
  }
  auto wv = [&](int i, int e) { return to_f32(reinterpret_cast<const TW *>(&wraw[i])[e]); };

  const int64_t gstep = (int64_t)gridDim.x * kWaves;
  int64_t row = (int64_t)blockIdx.x * kWaves + wave;
  // The next row's vectors are loaded into the registers of the current
  // row's as its dx leaves (vector i right after dx's vector i is stored), so
  // the next row's loads and this row's stores are in flight together.
  u32x4 cx[NV], cd[NV];
  auto load_vec = [&](int64_t rr, int i) {
    const int c = (i * 64 + lane) * VEC;
    if (c < n) {
      cx[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(x + rr * xs + c));
      cd[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(dy + rr * dys + c));
    }
  };
  float r = 0.f;
  if (row < rows) {
#pragma unroll
    for (int i = 0; i < NV; ++i) load_vec(row, i);
    r = rstd[row];
  }
#pragma unroll 1
  for (; row < rows; row += gstep) {
    const int64_t nrow = row + gstep;
    const bool more = nrow < rows;  // uniform over the wave
    const float rn = more ? rstd[nrow] : 0.f;
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * 64 + lane) * VEC;
      if (c < n) {
        const TX *ex = reinterpret_cast<const TX *>(&cx[i]);
        const TX *ed = reinterpret_cast<const TX *>(&cd[i]);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float xh = to_f32(ex[e]) * r, dv = to_f32(ed[e]);
          dot += dv * wv(i, e) * xh;
          acc[i][e] += dv * xh;
        }
      }
    }
    dot = wave_sum_full(dot) * inv_n;
    // Re-widen from the raw vectors instead of keeping 2*NV*VEC floats live
    // across the reduction (the empty asm stops the compiler from reusing the
    // first pass's values).
#pragma unroll
    for (int i = 0; i < NV; ++i) asm volatile("" : "+v"(cx[i]), "+v"(cd[i]));
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * 64 + lane) * VEC;
      if (c < n) {
        const TX *ex = reinterpret_cast<const TX *>(&cx[i]);
        const TX *ed = reinterpret_cast<const TX *>(&cd[i]);
        float o[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float xh = to_f32(ex[e]) * r;
          o[e] = r * (to_f32(ed[e]) * wv(i, e) - xh * dot);
        }
        store16_nt<TX>(dx + row * dxs + c, o);
      }
      if (more) load_vec(nrow, i);
    }
    r = rn;
  }
  // Cross-wave reduction of the dw partial (columns are lane-private).
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int e = 0; e < VEC; ++e) red[wave - 1][(i * VEC + e) * 64 + lane] = acc[i][e];
  }
  __syncthreads();
  if (wave == 0) {
    float *out = partial + (int64_t)blockIdx.x * n;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * 64 + lane) * VEC;
      if (c < n) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          float s = acc[i][e];
#pragma unroll
          for (int k = 0; k < kWaves - 1; ++k) s += red[k][(i * VEC + e) * 64 + lane];
          out[c + e] = s;
        }
      }
    }
  }
}

template <typename TX, typename TW>
__global__ __launch_bounds__(kThreads) void rmsnorm_bwd_loop(
    const TX *__restrict__ dy, int64_t dys, const TX *__restrict__ x, int64_t xs,
    const TW *__restrict__ w, const float *__restrict__ rstd, TX *__restrict__ dx, int64_t dxs,
    float *__restrict__ partial, int64_t rows, int n, int rows_per_wg) {
  // Columns strided over all 256 threads; rows walked sequentially by the
  // whole workgroup, with the row dot product reduced through LDS.
  __shared__ float red[kWaves];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const float inv_n = 1.0f / (float)n;
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_wg;
  const int64_t r1 = r0 + rows_per_wg < rows ? r0 + rows_per_wg : rows;
  float *out = partial + (int64_t)blockIdx.x * n;
  for (int c = threadIdx.x; c < n; c += kThreads) out[c] = 0.f;
  __syncthreads();
  for (int64_t row = r0; row < r1; ++row) {
    const float r = rstd[row];
    float dot = 0.f;
    for (int c = threadIdx.x; c < n; c += kThreads)
      dot += to_f32(dy[row * dys + c]) * to_f32(w[c]) * to_f32(x[row * xs + c]) * r;
    dot = wave_sum_full(dot);
    if (lane == 0) red[wave] = dot;
    __syncthreads();
    dot = 0.f;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) dot += red[k];
    dot *= inv_n;
    __syncthreads();
    for (int c = threadIdx.x; c < n; c += kThreads) {
      const float xh = to_f32(x[row * xs + c]) * r;
      const float d = to_f32(dy[row * dys + c]);
      const float g = d * to_f32(w[c]);
      dx[row * dxs + c] = from_f32<TX>(r * (g - xh * dot));
      out[c] += d * xh;  // column c is private to this thread
    }
  }
}

// dw[c] = sum_p partial[p, c]: 64 columns x 16 partial-row groups per block,
// each thread with four independent accumulators.  The loads of eight
// iterations are issued before their sums (one memory round trip for the 512
// partial rows of the usual plan instead of eight); the additions keep the
// order of the one-iteration loop.
template <typename TW>
__global__ __launch_bounds__(1024) void rmsnorm_dw_reduce(const float *__restrict__ partial,
                                                          TW *__restrict__ dw, int nparts, int n) {
  __shared__ float red[16][64];
  const int lane = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int col = blockIdx.x * 64 + lane;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  if (col < n) {
    int p = grp;
    for (; p + 64 * 7 + 48 < nparts; p += 64 * 8) {
      float v[8][4];
#pragma unroll
      for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int q = 0; q < 4; ++q) v[k][q] = partial[(int64_t)(p + 64 * k + 16 * q) * n + col];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        s0 += v[k][0];
        s1 += v[k][1];
        s2 += v[k][2];
        s3 += v[k][3];
      }
    }
    for (; p + 48 < nparts; p += 64) {
      s0 += partial[(int64_t)p * n + col];
      s1 += partial[(int64_t)(p + 16) * n + col];
      s2 += partial[(int64_t)(p + 32) * n + col];
      s3 += partial[(int64_t)(p + 48) * n + col];
    }
    for (; p < nparts; p += 16) s0 += partial[(int64_t)p * n + col];
  }
  red[grp][lane] = (s0 + s1) + (s2 + s3);
  __syncthreads();
  if (grp == 0 && col < n) {
    float t = 0.f;
#pragma unroll
    for (int g = 0; g < 16; ++g) t += red[g][lane];
    dw[col] = from_f32<TW>(t);
  }
}

// ---------------------------------------------------------------- dispatch
struct BwdPlan {
  int rows_per_wg;
  int nwg;
};

BwdPlan bwd_plan(int64_t rows) {
  // Aim for 512 workgroups: one resident round at two 4-wave workgroups per
  // CU (the register-resident backward runs two waves per SIMD); measured
  // at [32768, 4096] bf16: 512 -> 4.98 TB/s, 768 -> 4.21, 1024 -> 4.78,
  // 2048 -> 4.62.  The fp32 partial rows stay ~4% of the traffic.
  int64_t rpw = (rows + 511) / 512;
  if (rpw < 2 * kWaves) rpw = 2 * kWaves;
  BwdPlan p;
  p.rows_per_wg = (int)rpw;
  p.nwg = (int)((rows + rpw - 1) / rpw);
  if (p.nwg < 1) p.nwg = 1;
  return p;
}

// Number of 16-byte vectors per lane that a register-resident row needs,
// rounded up to the instantiated set; 0 when the row must stream.
template <typename TX>
int pick_nv(int64_t n, const void *a, int64_t a_stride, const void *b, int64_t b_stride,
            const void *c, int64_t c_stride) {
  constexpr int VEC = 16 / sizeof(TX);
  if (n % VEC) return 0;
  auto aligned = [](const void *p, int64_t stride) {
    return p == nullptr ||
           ((reinterpret_cast<uintptr_t>(p) % 16 == 0) && ((stride * (int64_t)sizeof(TX)) % 16 == 0));
  };
  if (!aligned(a, a_stride) || !aligned(b, b_stride) || !aligned(c, c_stride)) return 0;
  const int64_t need = (n + 64 * VEC - 1) / (64 * VEC);
  if (need <= 1) return 1;
  if (need <= 2) return 2;
  if (need <= 4) return 4;
  if (need <= 8) return 8;
  return 0;
}

template <typename TX, typename TW>
int fwd_typed(const void *x, int64_t xs, const void *w, void *y, int64_t ys, float *rstd,
              int64_t rows, int64_t n, float eps, hipStream_t st) {
  const TX *X = static_cast<const TX *>(x);
  const TW *W = static_cast<const TW *>(w);
  TX *Y = static_cast<TX *>(y);
  dim3 grid((unsigned)((rows + kWaves - 1) / kWaves));
  int nv = pick_nv<TX>(n, x, xs, y, ys, nullptr, 0);
  if (nv && (reinterpret_cast<uintptr_t>(w) % (16 / sizeof(TX) * sizeof(TW) >= 16 ? 16 : 8)) != 0)
    nv = 0;
  switch (nv) {
#define PB_FWD(NV)                                                                               \
  case NV:                                                                                       \
    hipLaunchKernelGGL((rmsnorm_fwd_reg<TX, TW, NV>), dim3(fwd_reg_grid(rows)), dim3(kThreads), \
                       0, st, X, xs, W, Y, ys, rstd, rows, (int)n, eps);                         \
    break;
    PB_FWD(1) PB_FWD(2) PB_FWD(4) PB_FWD(8)
#undef PB_FWD
    default:
      hipLaunchKernelGGL((rmsnorm_fwd_loop<TX, TW>), grid, dim3(kThreads), 0, st, X, xs, W, Y, ys,
                         rstd, rows, (int)n, eps);
  }
  return launch_status("pb_rmsnorm_fwd");
}

template <typename TX, typename TW>
int bwd_typed(const void *dy, int64_t dys, const void *x, int64_t xs, const void *w,
              const float *rstd, void *dx, int64_t dxs, void *dw, float *ws, int64_t rows,
              int64_t n, hipStream_t st) {
  const TX *DY = static_cast<const TX *>(dy);
  const TX *X = static_cast<const TX *>(x);
  const TW *W = static_cast<const TW *>(w);
  TX *DX = static_cast<TX *>(dx);
  BwdPlan p = bwd_plan(rows);
  int nv = pick_nv<TX>(n, x, xs, dy, dys, dx, dxs);
  if (nv && (reinterpret_cast<uintptr_t>(w) % (16 / sizeof(TX) * sizeof(TW) >= 16 ? 16 : 8)) != 0)
    nv = 0;
  dim3 grid(p.nwg);
  switch (nv) {
#define PB_BWD(NV)                                                                              \
  case NV:                                                                                      \
    hipLaunchKernelGGL((rmsnorm_bwd_reg<TX, TW, NV>), grid, dim3(kThreads), 0, st, DY, dys, X,  \
                       xs, W, rstd, DX, dxs, ws, rows, (int)n);                                 \
    break;
    PB_BWD(1) PB_BWD(2) PB_BWD(4) PB_BWD(8)
#undef PB_BWD
    default:
      hipLaunchKernelGGL((rmsnorm_bwd_loop<TX, TW>), grid, dim3(kThreads), 0, st, DY, dys, X, xs,
                         W, rstd, DX, dxs, ws, rows, (int)n, p.rows_per_wg);
  }
  int s = launch_status("pb_rmsnorm_bwd");
  if (s) return s;
  hipLaunchKernelGGL((rmsnorm_dw_reduce<TW>), dim3((unsigned)((n + 63) / 64)), dim3(1024), 0, st,
                     ws, static_cast<TW *>(dw), p.nwg, (int)n);
  return launch_status("pb_rmsnorm_bwd(dw)");
}

template <typename TX>
int fwd_w(int wdt, const void *x, int64_t xs, const void *w, void *y, int64_t ys, float *rstd,
          int64_t rows, int64_t n, float eps, hipStream_t st) {
  switch (wdt) {
    case PB_F32: return fwd_typed<TX, float>(x, xs, w, y, ys, rstd, rows, n, eps, st);
    case PB_BF16: return fwd_typed<TX, bf16_t>(x, xs, w, y, ys, rstd, rows, n, eps, st);
    default: return fwd_typed<TX, f16_t>(x, xs, w, y, ys, rstd, rows, n, eps, st);
  }
}

template <typename TX>
int bwd_w(int wdt, const void *dy, int64_t dys, const void *x, int64_t xs, const void *w,
          const float *rstd, void *dx, int64_t dxs, void *dw, float *ws, int64_t rows, int64_t n,
          hipStream_t st) {
  switch (wdt) {
    case PB_F32: return bwd_typed<TX, float>(dy, dys, x, xs, w, rstd, dx, dxs, dw, ws, rows, n, st);
    case PB_BF16: return bwd_typed<TX, bf16_t>(dy, dys, x, xs, w, rstd, dx, dxs, dw, ws, rows, n, st);
    default: return bwd_typed<TX, f16_t>(dy, dys, x, xs, w, rstd, dx, dxs, dw, ws, rows, n, st);
  }
}

// dw = 0 for an empty batch (a kernel, not a memset, so graph capture records no
// memset node).
__global__ __launch_bounds__(256) void rmsnorm_dw_zero(char *dw, int bytes_per, int64_t n) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= n) return;
  if (bytes_per == 4)
    reinterpret_cast<float *>(dw)[c] = 0.f;
  else
    reinterpret_cast<uint16_t *>(dw)[c] = 0;
}

}  // namespace
}  // namespace pb

extern "C" int pb_rmsnorm_fwd(const void *x, int64_t x_row_stride, int x_dtype, const void *w,
                              int w_dtype, void *y, int64_t y_row_stride, float *rstd,
                              int64_t rows, int64_t n, float eps, void *stream) {
  using namespace pb;
  clear_error();
  PB_CHECK_ARG(valid_dtype(x_dtype) && valid_dtype(w_dtype), "pb_rmsnorm_fwd: bad dtype");
  PB_CHECK_ARG(rows >= 0 && n > 0, "pb_rmsnorm_fwd: bad shape rows=%lld n=%lld", (long long)rows,
               (long long)n);
  PB_CHECK_SUPPORTED(n <= 65536, "RMSNorm feature dimension is too large for this kernel");
  PB_CHECK_ARG(x_row_stride >= n && y_row_stride >= n, "pb_rmsnorm_fwd: row stride < n");
  if (rows == 0) return PB_OK;
  hipStream_t st = as_stream(stream);
  switch (x_dtype) {
    case PB_F32: return fwd_w<float>(w_dtype, x, x_row_stride, w, y, y_row_stride, rstd, rows, n, eps, st);
    case PB_BF16: return fwd_w<bf16_t>(w_dtype, x, x_row_stride, w, y, y_row_stride, rstd, rows, n, eps, st);
    default: return fwd_w<f16_t>(w_dtype, x, x_row_stride, w, y, y_row_stride, rstd, rows, n, eps, st);
  }
}

extern "C" int64_t pb_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t n) {
  if (rows <= 0 || n <= 0) return 0;
  return (int64_t)pb::bwd_plan(rows).nwg * n * (int64_t)sizeof(float);
}

extern "C" int pb_rmsnorm_bwd(const void *dy, int64_t dy_row_stride, const void *x,
                              int64_t x_row_stride, int x_dtype, const void *w, int w_dtype,
                              const float *rstd, void *dx, int64_t dx_row_stride, void *dw,
                              void *workspace, int64_t rows, int64_t n, void *stream) {
  using namespace pb;
  clear_error();
  PB_CHECK_ARG(valid_dtype(x_dtype) && valid_dtype(w_dtype), "pb_rmsnorm_bwd: bad dtype");
  PB_CHECK_ARG(rows >= 0 && n > 0, "pb_rmsnorm_bwd: bad shape");
  PB_CHECK_SUPPORTED(n <= 65536, "RMSNorm feature dimension is too large for this kernel");
  PB_CHECK_ARG(x_row_stride >= n && dy_row_stride >= n && dx_row_stride >= n,
               "pb_rmsnorm_bwd: row stride < n");
  hipStream_t st = as_stream(stream);
  if (rows == 0) {
    // dw of an empty batch is zero.
    PB_CHECK_ARG(dw != nullptr, "pb_rmsnorm_bwd: null dw");
    hipLaunchKernelGGL(rmsnorm_dw_zero, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       static_cast<char *>(dw), dtype_bytes(w_dtype), n);
    return launch_status("pb_rmsnorm_bwd(empty)");
  }
  PB_CHECK_ARG(workspace != nullptr, "pb_rmsnorm_bwd: workspace is required");
  float *ws = static_cast<float *>(workspace);
  switch (x_dtype) {
    case PB_F32: return bwd_w<float>(w_dtype, dy, dy_row_stride, x, x_row_stride, w, rstd, dx, dx_row_stride, dw, ws, rows, n, st);
    case PB_BF16: return bwd_w<bf16_t>(w_dtype, dy, dy_row_stride, x, x_row_stride, w, rstd, dx, dx_row_stride, dw, ws, rows, n, st);
    default: return bwd_w<f16_t>(w_dtype, dy, dy_row_stride, x, x_row_stride, w, rstd, dx, dx_row_stride, dw, ws, rows, n, st);
  }
}

// ---------------------------------------------------------------- allocation-free backward
// pb_rmsnorm_bwd for callers that can neither allocate nor pass a workspace:
// the dW partial rows live in a file-scope device array, one copy per GPU.
// In host code `scratch` names a host-side stand-in, never the device memory:
// its device address is looked up once per device (hipGetSymbolAddress, with
// that device current) and only that address reaches a kernel.  Every
// partial row is fully written by the backward kernel before the reduction
// reads it, so nothing needs clearing between calls; calls that overlap on
// one GPU (two streams, two threads) race on the array.
static __device__ __align__(256) float scratch[PB_RMSNORM_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace pb {
namespace {

constexpr int64_t kNoAllocScratchBytes = PB_RMSNORM_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

std::once_flag g_scratch_once[kMaxDevices];
float *g_scratch_ptr[kMaxDevices] = {};
hipError_t g_scratch_err[kMaxDevices] = {};

// Device address of this device's scratch array (found on the first call made
// with `dev` current; later calls reuse it).
int scratch_on(int dev, float **out) {
  PB_CHECK_SUPPORTED(dev >= 0 && dev < kMaxDevices, "pb_rmsnorm_bwd_noalloc: device %d out of range",
                     dev);
  std::call_once(g_scratch_once[dev], [dev] {
    g_scratch_err[dev] = hipGetSymbolAddress(reinterpret_cast<void **>(&g_scratch_ptr[dev]),
                                             HIP_SYMBOL(scratch));
  });
  if (g_scratch_err[dev] != hipSuccess || g_scratch_ptr[dev] == nullptr) {
    set_error("pb_rmsnorm_bwd_noalloc: hipGetSymbolAddress failed on device %d: %s", dev,
              hipGetErrorString(g_scratch_err[dev]));
    return PB_EHIP;
  }
  *out = g_scratch_ptr[dev];
  return PB_OK;
}

}  // namespace
}  // namespace pb

extern "C" int pb_rmsnorm_bwd_noalloc(const void *dy, int64_t dy_row_stride, const void *x,
                                      int64_t x_row_stride, int x_dtype, const void *w,
                                      int w_dtype, const float *rstd, void *dx,
                                      int64_t dx_row_stride, void *dw, int64_t rows, int64_t n,
                                      void *stream) {
  using namespace pb;
  clear_error();
  PB_CHECK_ARG(rows >= 0 && n > 0, "pb_rmsnorm_bwd_noalloc: bad shape");
  const int64_t need = pb_rmsnorm_bwd_workspace_bytes(rows, n);
  PB_CHECK_SUPPORTED(need <= kNoAllocScratchBytes,
                     "pb_rmsnorm_bwd_noalloc: rows=%lld n=%lld need %lld bytes of dW partials, "
                     "more than the %lld-byte static scratch (use pb_rmsnorm_bwd with a workspace)",
                     (long long)rows, (long long)n, (long long)need,
                     (long long)kNoAllocScratchBytes);
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("pb_rmsnorm_bwd_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return PB_EHIP;
  }
  float *ws = nullptr;
  if (int rc = scratch_on(dev, &ws)) return rc;
  return pb_rmsnorm_bwd(dy, dy_row_stride, x, x_row_stride, x_dtype, w, w_dtype, rstd, dx,
                        dx_row_stride, dw, ws, rows, n, stream);
}
