// Fused LM-head cross-entropy for gfx950: logits = x W^T are never stored.
//
// Reference: packbalance/kernels/fused_ce.py:143-217 (_FusedLinearCE,
// linear_cross_entropy) -- the SUM over rows with target != ignore_index of
//     lse(x_n W^T) - x_n . w_t + z * lse^2,
// gradients dlogits = softmax*(1 + 2z*lse) - onehot (fused_ce.py:80-84),
// dx = dlogits W, dW = dlogits^T x, both scaled by grad_output.
//
// Everything runs on one bf16 MFMA GEMM tile, C[m][n] = sum_k A[m][k] B[n][k]
// (both operands K-contiguous, "NT"), 128 x 128 x 64 per workgroup, four waves
// of 64 x 64 (2 x 2 v_mfma_f32_32x32x16_bf16 blocks), register-prefetched
// double buffering through LDS.  Four epilogues:
//   kLse      A = W, B = x: C = logits^T, lane <-> token.  Per token, a
//             (max, sum exp) partial over the tile's 128 vocab rows and the
//             target logit; the [tokens x vocab] tile is discarded.
//   kDlogits  same product over one vocab chunk; writes dlogits (scaled by the
//             device-resident grad_output) as dL [tokens][chunk] and dL^T.
//   kAccum    dx += dL W_chunk (fp32 accumulator; the last chunk writes x's dtype).
//   kStore    dW_chunk = dL^T x (written in W's dtype, or added to an fp32 dW).
// A small kernel merges the forward partials into lse / per-row loss, and a
// single workgroup sums the rows in a fixed order (deterministic scalar).
#include <math.h>

#include "common.hpp"

namespace pb {
namespace ce {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int AP = BK + 8;  // LDS row pitch (elements): 144 bytes, 16-byte aligned rows

enum Mode { kLse = 0, kDlogits = 1, kAccum = 2, kStore = 3 };

struct GemmArgs {
  const bf16_t *A;  // [M][K], row stride lda
  const bf16_t *B;  // [N][K], row stride ldb
  int64_t lda, ldb;
  int M, N, K;
  // kLse / kDlogits: m = vocab row (offset v0 into the full vocab), n = token
  int v0, V;
  const int64_t *targets;
  int64_t ignore_index;
  float z;
  float *part_m, *part_s;  // kLse: [nMT][N] partials (log2 domain)
  float *tgt;              // kLse: [N] target logits
  const float *lse;        // kDlogits: [N] natural-log lse
  const float *grad_out;   // kDlogits: device scalar
  bf16_t *dl;              // kDlogits: [N][ldl] (token-major)
  bf16_t *dlt;             // kDlogits: [M][ldlt] (vocab-major)
  int64_t ldl, ldlt;
  // kAccum / kStore
  float *acc;     // kAccum: fp32 [M][N] accumulator, row stride ldc
  void *out;      // kAccum (last) / kStore: output, row stride ldo
  int64_t ldc, ldo;
  int out_dtype;
  int first, last;
  int accum_out;  // kStore: out is fp32 and the product is added to it
  // kAccum split-K: blockIdx.y = split; each split covers k_per_split of K and
  // writes fp32 partials part[split][M][N]; split_reduce folds them.
  int k_per_split;
  float *part;
};

__device__ __forceinline__ f32x16_t zero16() {
  f32x16_t z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Eight K-consecutive elements of one operand row starting at column k; zero
// outside the matrix.  The full 16-byte load is used when all eight lie below
// K, the K tail is read element by element.
__device__ __forceinline__ bf16x8_t load8(const bf16_t *row, int k, int K, bool row_ok) {
  bf16x8_t r;
  if (row_ok && k + 8 <= K) {
    u32x4 raw = *reinterpret_cast<const u32x4 *>(row + k);
    return *reinterpret_cast<bf16x8_t *>(&raw);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (row_ok && k + i < K) ? row[k + i] : (bf16_t)0.0f;
  return r;
}

__device__ __forceinline__ void store_out(void *out, int dtype, int64_t idx, float v) {
  if (dtype == PB_F32)
    static_cast<float *>(out)[idx] = v;
  else if (dtype == PB_BF16)
    static_cast<bf16_t *>(out)[idx] = (bf16_t)v;
  else
    static_cast<f16_t *>(out)[idx] = (f16_t)v;
}

// kDlogits stages its bf16 tile [BM][TP] (vocab-major) in the operand LDS
// after the main loop, so both dlogits layouts leave as 16-byte stores.
constexpr int TP = BN + 8;  // staging row pitch (elements): 272 bytes
static_assert(BM * TP * 2 <= 2 * BM * AP * 2, "staging tile must fit the operand LDS");

template <int MODE>
__global__ __launch_bounds__(256) void gemm_nt(GemmArgs g) {
  __shared__ __align__(16) bf16_t smem[(BM + BN) * AP];
  bf16_t *const As = smem;
  bf16_t *const Bs = smem + BM * AP;
  __shared__ float red_m[2][BN], red_s[2][BN];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hh = lane >> 5, l32 = lane & 31;
  const int wm = wave >> 1, wn = wave & 1;

  // Tile order: tiles sharing a B (token/column) panel are consecutive, so a
  // column panel stays hot in L2 while the A panels stream past it.
  const int ntm = (g.M + BM - 1) / BM;
  const int tm = blockIdx.x % ntm, tn = blockIdx.x / ntm;
  const int m0 = tm * BM, n0 = tn * BN;
  // K range of this workgroup (all of K unless split-K).
  const int kb = MODE == kAccum && g.part ? blockIdx.y * g.k_per_split : 0;
  const int ke = MODE == kAccum && g.part ? min(g.K, kb + g.k_per_split) : g.K;

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero16();

  // Each thread moves 4 + 4 sixteen-byte chunks per K tile.
  bf16x8_t ra[4], rb[4];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 3, kc = (c & 7) * 8;
      const int k = k0 + kc;
      const int am = m0 + row, bn = n0 + row;
      ra[i] = load8(g.A + (int64_t)(am < g.M ? am : 0) * g.lda, k, ke, am < g.M);
      rb[i] = load8(g.B + (int64_t)(bn < g.N ? bn : 0) * g.ldb, k, ke, bn < g.N);
    }
  };

  const int nk = (ke - kb + BK - 1) / BK;
  fetch(kb);
  for (int kt = 0; kt < nk; ++kt) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 3, kc = (c & 7) * 8;
      *reinterpret_cast<bf16x8_t *>(&As[row * AP + kc]) = ra[i];
      *reinterpret_cast<bf16x8_t *>(&Bs[row * AP + kc]) = rb[i];
    }
    __syncthreads();
    if (kt + 1 < nk) fetch(kb + (kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8_t a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *reinterpret_cast<const bf16x8_t *>(
            &As[(64 * wm + 32 * i + l32) * AP + 16 * ks + 8 * hh]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = *reinterpret_cast<const bf16x8_t *>(
            &Bs[(64 * wn + 32 * j + l32) * AP + 16 * ks + 8 * hh]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }

  // C layout: block (i, j), register r -> row m = 64wm + 32i + 8(r/4) + 4hh + r%4,
  // column n = 64wn + 32j + l32.
  if constexpr (MODE == kLse || MODE == kDlogits) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int nl = 64 * wn + 32 * j + l32;
      const int n = n0 + nl;
      const bool nvalid = n < g.N;
      const int64_t t = nvalid ? g.targets[n] : g.ignore_index;
      const bool valid = t != g.ignore_index;
      if constexpr (MODE == kLse) {
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * hh + (r & 3);
            const float x = acc[i][j][r];
            if (m < g.M) {
              mx = fmaxf(mx, x);
              if (valid && nvalid && (int64_t)(g.v0 + m) == t) g.tgt[n] = x;
            }
          }
        mx *= kLog2e;
        float sm = 0.f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * hh + (r & 3);
            if (m < g.M) sm += fast_exp2(acc[i][j][r] * kLog2e - mx);
          }
        // Merge the two lane halves (other 4-row groups), then the two wave rows.
        const float mo = __shfl_xor(mx, 32), so = __shfl_xor(sm, 32);
        const float mn = fmaxf(mx, mo);
        if (mn != -INFINITY) sm = sm * fast_exp2(mx - mn) + so * fast_exp2(mo - mn);
        mx = mn;
        if (hh == 0) {
          red_m[wm][nl] = mx;
          red_s[wm][nl] = sm;
        }
      } else {
        // dlogits of this lane's token into the staging tile (vocab-major);
        // padding rows / columns (m >= M, n >= N) hold 0.
        if (j == 0) __syncthreads();  // every wave is done with the operand LDS
        const float lse = nvalid ? g.lse[n] : 0.f;
        const float lse2 = lse * kLog2e;
        const float scale = valid ? (*g.grad_out) * (1.0f + 2.0f * g.z * lse) : 0.f;
        const float one = valid ? (*g.grad_out) : 0.f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int ml = 64 * wm + 32 * i + 8 * (r >> 2) + 4 * hh + (r & 3);
            const int m = m0 + ml;
            float gv = fast_exp2(acc[i][j][r] * kLog2e - lse2) * scale;
            if ((int64_t)(g.v0 + m) == t) gv -= one;
            smem[ml * TP + nl] = (bf16_t)(m < g.M && nvalid ? gv : 0.f);
          }
      }
    }
    if constexpr (MODE == kDlogits) {
      __syncthreads();
      // dL^T [vocab][tokens]: 16 threads per 256-byte staging row.
#pragma unroll
      for (int k = 0; k < BM * (BN / 8) / 256; ++k) {
        const int c = tid + 256 * k;
        const int ml = c >> 4, n8 = (c & 15) * 8;
        if (m0 + ml < g.M && n0 + n8 < g.N)
          *reinterpret_cast<u32x4 *>(g.dlt + (int64_t)(m0 + ml) * g.ldlt + n0 + n8) =
              *reinterpret_cast<const u32x4 *>(&smem[ml * TP + n8]);
      }
      // dL [tokens][vocab]: lane <-> token (conflict-free column reads), eight
      // vocab rows per 16-byte store.
#pragma unroll
      for (int k = 0; k < (BM / 8) * BN / 256; ++k) {
        const int nl = tid & (BN - 1), m8 = 8 * ((tid >> 7) + 2 * k);
        if (n0 + nl < g.N && m0 + m8 < g.M) {
          bf16x8_t v;
#pragma unroll
          for (int x = 0; x < 8; ++x) v[x] = smem[(m8 + x) * TP + nl];
          *reinterpret_cast<bf16x8_t *>(g.dl + (int64_t)(n0 + nl) * g.ldl + m0 + m8) = v;
        }
      }
    }
    if constexpr (MODE == kLse) {
      __syncthreads();
      if (tid < BN) {
        const int n = n0 + tid;
        float m1 = red_m[0][tid], s1 = red_s[0][tid];
        const float m2 = red_m[1][tid], s2 = red_s[1][tid];
        const float mn = fmaxf(m1, m2);
        if (mn != -INFINITY) s1 = s1 * fast_exp2(m1 - mn) + s2 * fast_exp2(m2 - mn);
        if (n < g.N) {
          g.part_m[(int64_t)tm * g.N + n] = mn;
          g.part_s[(int64_t)tm * g.N + n] = s1;
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = n0 + 64 * wn + 32 * j + l32;
        if (n >= g.N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (m >= g.M) continue;
          float v = acc[i][j][r];
          if constexpr (MODE == kAccum) {
            if (g.part) {
              g.part[((int64_t)blockIdx.y * g.M + m) * g.N + n] = v;
              continue;
            }
            float *p = g.acc + (int64_t)m * g.ldc + n;
            if (!g.first) v += *p;
            if (g.last)
              store_out(g.out, g.out_dtype, (int64_t)m * g.ldo + n, v);
            else
              *p = v;
          } else {
            if (MODE == kStore && g.accum_out) {
              static_cast<float *>(g.out)[(int64_t)m * g.ldo + n] += v;
              continue;
            }
            store_out(g.out, g.out_dtype, (int64_t)m * g.ldo + n, v);
          }
        }
      }
  }
}

// out (+)= sum of the split-K partials (the kAccum epilogue, applied after a
// split-K GEMM): fp32 accumulator in between chunks, out dtype at the end.
__global__ __launch_bounds__(256) void split_reduce(GemmArgs g, int splits) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)g.M * g.N) return;
  const int m = (int)(t / g.N), n = (int)(t - (t / g.N) * g.N);
  float v = 0.f;
  for (int sidx = 0; sidx < splits; ++sidx) v += g.part[(int64_t)sidx * g.M * g.N + t];
  float *p = g.acc + (int64_t)m * g.ldc + n;
  if (!g.first) v += *p;
  if (g.last)
    store_out(g.out, g.out_dtype, (int64_t)m * g.ldo + n, v);
  else
    *p = v;
}

// Merge the per-tile partials of every token: lse (natural log) and row loss.
// Block = 64 tokens x 16 partial-tile groups; the 16 groups are merged in LDS.
__global__ __launch_bounds__(1024) void lse_combine(const float *__restrict__ part_m,
                                                    const float *__restrict__ part_s, int ntiles,
                                                    int n, const float *__restrict__ tgt,
                                                    const int64_t *__restrict__ targets,
                                                    int64_t ignore_index, int v, float z,
                                                    float *__restrict__ lse_out,
                                                    float *__restrict__ loss) {
  __shared__ float rm[16][64], rs[16][64];
  const int lane = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int i = blockIdx.x * 64 + lane;
  float m = -INFINITY, s = 0.f;
  if (i < n) {
    for (int t = grp; t < ntiles; t += 16) {
      const float m2 = part_m[(int64_t)t * n + i], s2 = part_s[(int64_t)t * n + i];
      const float mn = fmaxf(m, m2);
      if (mn == -INFINITY) continue;
      s = s * fast_exp2(m - mn) + s2 * fast_exp2(m2 - mn);
      m = mn;
    }
  }
  rm[grp][lane] = m;
  rs[grp][lane] = s;
  __syncthreads();
  if (grp != 0 || i >= n) return;
  for (int g = 1; g < 16; ++g) {
    const float m2 = rm[g][lane], s2 = rs[g][lane];
    const float mn = fmaxf(m, m2);
    if (mn == -INFINITY) continue;
    s = s * fast_exp2(m - mn) + s2 * fast_exp2(m2 - mn);
    m = mn;
  }
  const float lse = (m + log2f(s)) * kLn2;
  lse_out[i] = lse;
  const int64_t t = targets[i];
  float l = 0.f;
  if (t != ignore_index) l = (t < 0 || t >= v) ? NAN : lse - tgt[i] + z * lse * lse;
  loss[i] = l;
}

// Fixed-order sum of the row losses (one workgroup): deterministic scalar.
__global__ __launch_bounds__(1024) void sum_rows(const float *__restrict__ x, int n,
                                                 float *__restrict__ out) {
  __shared__ float red[16];
  float s = 0.f;
  for (int i = threadIdx.x; i < n; i += 1024) s += x[i];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (int w = 0; w < 16; ++w) t += red[w];
    *out = t;
  }
}

// dst[c][r] = src[r][c] (bf16 out), src of any float dtype; 64 x 64 LDS tiles.
// Also used with transpose = 0 as a plain cast/copy into a padded buffer.
template <typename T, bool TRANSPOSE>
__global__ __launch_bounds__(256) void pack_bf16(const T *__restrict__ src, int64_t lds, int rows,
                                                 int cols, bf16_t *__restrict__ dst, int64_t ldd,
                                                 int drows, int dcols) {
  __shared__ bf16_t tile[64][66];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  if constexpr (TRANSPOSE) {
    for (int y = ty; y < 64; y += 4) {
      const int r = r0 + y, c = c0 + tx;
      tile[y][tx] = (r < rows && c < cols) ? (bf16_t)to_f32(src[(int64_t)r * lds + c]) : (bf16_t)0.0f;
    }
    __syncthreads();
    // Output row = source column; zero-fill the padded region.
    for (int y = ty; y < 64; y += 4) {
      const int orow = c0 + y, ocol = r0 + tx;
      if (orow < drows && ocol < dcols) dst[(int64_t)orow * ldd + ocol] = tile[tx][y];
    }
  } else {
    for (int y = ty; y < 64; y += 4) {
      const int r = r0 + y, c = c0 + tx;
      if (r < drows && c < dcols)
        dst[(int64_t)r * ldd + c] =
            (r < rows && c < cols) ? (bf16_t)to_f32(src[(int64_t)r * lds + c]) : (bf16_t)0.0f;
    }
  }
}

unsigned tiles(int m, int n) { return (unsigned)(((m + BM - 1) / BM) * ((n + BN - 1) / BN)); }

}  // namespace ce
}  // namespace pb

using pb::bf16_t;

namespace {
bool k_aligned(const void *p, int64_t ld) {
  return (reinterpret_cast<uintptr_t>(p) % 16) == 0 && (ld % 8) == 0;
}
}  // namespace

extern "C" int pb_pack_bf16(const void *src, int src_dtype, int64_t src_ld, int64_t rows,
                            int64_t cols, void *dst, int64_t dst_ld, int64_t dst_rows,
                            int64_t dst_cols, int transpose, void *stream) {
  using namespace pb;
  clear_error();
  PB_CHECK_ARG(valid_dtype(src_dtype), "pb_pack_bf16: bad dtype");
  PB_CHECK_ARG(rows >= 0 && cols >= 0 && dst_rows >= 0 && dst_cols >= 0 && src_ld >= cols &&
                   dst_ld >= dst_cols,
               "pb_pack_bf16: bad shape");
  PB_CHECK_SUPPORTED(rows < (1LL << 31) && cols < (1LL << 31), "pb_pack_bf16: too large");
  if (dst_rows == 0 || dst_cols == 0) return PB_OK;
  hipStream_t st = as_stream(stream);
  // Grid covers the destination (transpose: source cols -> dest rows).
  const int64_t grid_r = transpose ? dst_cols : dst_rows, grid_c = transpose ? dst_rows : dst_cols;
  dim3 grid((unsigned)((grid_c + 63) / 64), (unsigned)((grid_r + 63) / 64));
  bf16_t *D = static_cast<bf16_t *>(dst);
#define PB_PACK(T)                                                                                  \
  if (transpose)                                                                                    \
    hipLaunchKernelGGL((ce::pack_bf16<T, true>), grid, dim3(256), 0, st, static_cast<const T *>(src), \
                       src_ld, (int)rows, (int)cols, D, dst_ld, (int)dst_rows, (int)dst_cols);      \
  else                                                                                              \
    hipLaunchKernelGGL((ce::pack_bf16<T, false>), grid, dim3(256), 0, st, static_cast<const T *>(src), \
                       src_ld, (int)rows, (int)cols, D, dst_ld, (int)dst_rows, (int)dst_cols);
  if (src_dtype == PB_F32) {
    PB_PACK(float)
  } else if (src_dtype == PB_BF16) {
    PB_PACK(bf16_t)
  } else {
    PB_PACK(f16_t)
  }
#undef PB_PACK
  return launch_status("pb_pack_bf16");
}

extern "C" int64_t pb_lmhead_ce_workspace_bytes(int64_t n, int64_t v) {
  if (n <= 0 || v <= 0) return 0;
  const int64_t nmt = (v + pb::ce::BM - 1) / pb::ce::BM;
  return (2 * nmt * n + n) * (int64_t)sizeof(float);  // partial m, s; target logits
}

extern "C" int pb_lmhead_ce_fwd(const void *x, int64_t ldx, const void *w, int64_t ldw,
                                int64_t n, int64_t v, int64_t d, const int64_t *targets,
                                int64_t ignore_index, float z_loss_coeff, float *loss_rows,
                                float *lse, float *loss_sum, void *workspace, void *stream) {
  using namespace pb;
  using namespace pb::ce;
  clear_error();
  PB_CHECK_ARG(n >= 0 && v >= 1 && d >= 1, "pb_lmhead_ce_fwd: bad shape n=%lld v=%lld d=%lld",
               (long long)n, (long long)v, (long long)d);
  PB_CHECK_SUPPORTED(n < (1LL << 31) && v < (1LL << 31) && d < (1LL << 31),
                     "pb_lmhead_ce_fwd: too large");
  PB_CHECK_ARG(k_aligned(x, ldx) && k_aligned(w, ldw) && d % 8 == 0,
               "pb_lmhead_ce_fwd: x/w rows must be 16-byte aligned with d %% 8 == 0");
  hipStream_t st = as_stream(stream);
  if (n == 0) {
    // The fixed-order sum over no rows writes 0 (a kernel, so graph capture
    // records no memset node).
    hipLaunchKernelGGL(sum_rows, dim3(1), dim3(1024), 0, st, (const float *)nullptr, 0, loss_sum);
    return launch_status("pb_lmhead_ce_fwd(empty)");
  }
  const int nmt = (int)((v + BM - 1) / BM);
  float *ws = static_cast<float *>(workspace);
  GemmArgs g = {};
  g.A = static_cast<const bf16_t *>(w);
  g.lda = ldw;
  g.B = static_cast<const bf16_t *>(x);
  g.ldb = ldx;
  g.M = (int)v; g.N = (int)n; g.K = (int)d;
  g.v0 = 0; g.V = (int)v;
  g.targets = targets;
  g.ignore_index = ignore_index;
  g.z = z_loss_coeff;
  g.part_m = ws;
  g.part_s = ws + (int64_t)nmt * n;
  g.tgt = ws + 2 * (int64_t)nmt * n;
  hipLaunchKernelGGL(gemm_nt<kLse>, dim3(tiles(g.M, g.N)), dim3(256), 0, st, g);
  int rc = launch_status("pb_lmhead_ce_fwd(gemm)");
  if (rc) return rc;
  hipLaunchKernelGGL(lse_combine, dim3((unsigned)((n + 63) / 64)), dim3(1024), 0, st, g.part_m,
                     g.part_s, nmt, (int)n, g.tgt, targets, ignore_index, (int)v, z_loss_coeff, lse,
                     loss_rows);
  hipLaunchKernelGGL(sum_rows, dim3(1), dim3(1024), 0, st, loss_rows, (int)n, loss_sum);
  return launch_status("pb_lmhead_ce_fwd");
}

namespace {
// Backward workspace: dL [n][vchunk] bf16, dL^T [vchunk][n8] bf16, the fp32
// dx accumulator [n][d], the split-K partials [splits][n][d] (256-byte aligned
// pieces).
struct BwdWs {
  int64_t ldl, ldlt, off_dlt, off_acc, off_part, bytes;
  int splits, k_per_split;
};

BwdWs bwd_ws(int64_t n, int64_t v, int64_t d, int64_t vchunk) {
  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  BwdWs w;
  w.ldl = vchunk;
  w.ldlt = (n + 7) / 8 * 8;
  w.off_dlt = al(n * vchunk * 2);
  w.off_acc = w.off_dlt + al(vchunk * w.ldlt * 2);
  w.off_part = w.off_acc + al(n * d * 4);
  // Split the dx GEMM's K (vocab chunk) when its tile grid cannot fill the GPU.
  const int64_t tiles = ((n + pb::ce::BM - 1) / pb::ce::BM) * ((d + pb::ce::BN - 1) / pb::ce::BN);
  int64_t splits = (512 + tiles - 1) / tiles;
  const int64_t kmin = 1024;
  if (splits > vchunk / kmin) splits = vchunk / kmin;
  if (splits > 8) splits = 8;
  if (splits < 1) splits = 1;
  w.splits = (int)splits;
  w.k_per_split = (int)(((vchunk + splits - 1) / splits + pb::ce::BK - 1) / pb::ce::BK * pb::ce::BK);
  w.bytes = w.off_part + (splits > 1 ? al(splits * n * d * 4) : 0);
  return w;
}
}  // namespace

extern "C" int64_t pb_lmhead_ce_bwd_workspace_bytes(int64_t n, int64_t v, int64_t d,
                                                    int64_t vchunk) {
  if (n <= 0 || v <= 0 || d <= 0 || vchunk <= 0) return 0;
  return bwd_ws(n, v, d, vchunk).bytes;
}

extern "C" int pb_lmhead_ce_bwd(const void *x, int64_t ldx, const void *w, int64_t ldw,
                                const void *xt, int64_t ldxt, const void *wt, int64_t ldwt,
                                int64_t n, int64_t v, int64_t d, const int64_t *targets,
                                int64_t ignore_index, float z_loss_coeff, const float *lse,
                                const float *grad_out, int64_t vchunk, void *workspace, void *dx,
                                int dx_dtype, int64_t lddx, void *dw, int dw_dtype, int64_t lddw,
                                int dw_accumulate, void *stream) {
  using namespace pb;
  using namespace pb::ce;
  clear_error();
  PB_CHECK_ARG(n >= 1 && v >= 1 && d >= 1 && vchunk >= 1, "pb_lmhead_ce_bwd: bad shape");
  PB_CHECK_SUPPORTED(n < (1LL << 31) && v < (1LL << 31) && d < (1LL << 31),
                     "pb_lmhead_ce_bwd: too large");
  PB_CHECK_ARG(valid_dtype(dx_dtype) && valid_dtype(dw_dtype), "pb_lmhead_ce_bwd: bad dtype");
  PB_CHECK_ARG(vchunk % 8 == 0, "pb_lmhead_ce_bwd: vchunk must be a multiple of 8");
  PB_CHECK_ARG(!dw_accumulate || dw_dtype == PB_F32,
               "pb_lmhead_ce_bwd: dw_accumulate needs an fp32 dw");
  PB_CHECK_ARG(k_aligned(x, ldx) && k_aligned(w, ldw) && k_aligned(xt, ldxt) &&
                   k_aligned(wt, ldwt) && k_aligned(workspace, 8) && d % 8 == 0,
               "pb_lmhead_ce_bwd: operands must be 16-byte aligned with row strides %% 8 == 0");
  PB_CHECK_ARG(ldxt >= n && ldwt >= v && lddx >= d && lddw >= d,
               "pb_lmhead_ce_bwd: row strides too small");
  const BwdWs L = bwd_ws(n, v, d, vchunk);
  char *wsb = static_cast<char *>(workspace);
  bf16_t *dl = reinterpret_cast<bf16_t *>(wsb);
  bf16_t *dlt = reinterpret_cast<bf16_t *>(wsb + L.off_dlt);
  float *dx_acc = reinterpret_cast<float *>(wsb + L.off_acc);
  float *part = L.splits > 1 ? reinterpret_cast<float *>(wsb + L.off_part) : nullptr;
  const int64_t ldl = L.ldl, ldlt = L.ldlt;
  hipStream_t st = as_stream(stream);
  const int64_t nchunks = (v + vchunk - 1) / vchunk;
  for (int64_t c = 0; c < nchunks; ++c) {
    const int64_t v0 = c * vchunk;
    const int vc = (int)((v - v0) < vchunk ? (v - v0) : vchunk);
    // 1) dlogits for vocab rows [v0, v0 + vc): dL [n][vc], dL^T [vc][n].
    GemmArgs g = {};
    g.A = static_cast<const bf16_t *>(w) + v0 * ldw;
    g.lda = ldw;
    g.B = static_cast<const bf16_t *>(x);
    g.ldb = ldx;
    g.M = vc; g.N = (int)n; g.K = (int)d;
    g.v0 = (int)v0; g.V = (int)v;
    g.targets = targets;
    g.ignore_index = ignore_index;
    g.z = z_loss_coeff;
    g.lse = lse;
    g.grad_out = grad_out;
    g.dl = dl;
    g.dlt = dlt;
    g.ldl = ldl;
    g.ldlt = ldlt;
    hipLaunchKernelGGL(gemm_nt<kDlogits>, dim3(tiles(g.M, g.N)), dim3(256), 0, st, g);
    int rc = launch_status("pb_lmhead_ce_bwd(dlogits)");
    if (rc) return rc;
    // 2) dx (+)= dL W_chunk: A = dL [n][vc], B = W^T[:, v0:v0+vc] rows d.
    GemmArgs gx = {};
    gx.A = dl;
    gx.lda = ldl;
    gx.B = static_cast<const bf16_t *>(wt) + v0;
    gx.ldb = ldwt;
    gx.M = (int)n; gx.N = (int)d; gx.K = vc;
    gx.acc = dx_acc;
    gx.ldc = d;
    gx.out = dx;
    gx.ldo = lddx;
    gx.out_dtype = dx_dtype;
    gx.first = c == 0;
    gx.last = c == nchunks - 1;
    gx.part = part;
    gx.k_per_split = L.k_per_split;
    const int splits = part ? (vc + L.k_per_split - 1) / L.k_per_split : 1;
    hipLaunchKernelGGL(gemm_nt<kAccum>, dim3(tiles(gx.M, gx.N), splits), dim3(256), 0, st, gx);
    if (part) {
      const int64_t cnt = (int64_t)gx.M * gx.N;
      hipLaunchKernelGGL(split_reduce, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, st, gx,
                         splits);
    }
    // 3) dW[v0:v0+vc] = dL^T x: A = dL^T [vc][n], B = x^T rows d.
    GemmArgs gw = {};
    gw.A = dlt;
    gw.lda = ldlt;
    gw.B = static_cast<const bf16_t *>(xt);
    gw.ldb = ldxt;
    gw.M = vc; gw.N = (int)d; gw.K = (int)n;
    gw.out = static_cast<char *>(dw) + v0 * lddw * (dw_dtype == PB_F32 ? 4 : 2);
    gw.ldo = lddw;
    gw.out_dtype = dw_dtype;
    gw.accum_out = dw_accumulate != 0;
    hipLaunchKernelGGL(gemm_nt<kStore>, dim3(tiles(gw.M, gw.N)), dim3(256), 0, st, gw);
    rc = launch_status("pb_lmhead_ce_bwd(dx/dw)");
    if (rc) return rc;
  }
  return PB_OK;
}
