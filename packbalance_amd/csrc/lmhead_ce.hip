// Fused LM-head cross-entropy for gfx950: logits = x W^T are either never
// stored (the backward recomputes them) or kept as bf16 for the backward.
//
// Reference: packbalance/kernels/fused_ce.py:143-217 (_FusedLinearCE,
// linear_cross_entropy) -- the SUM over rows with target != ignore_index of
//     lse(x_n W^T) - x_n . w_t + z * lse^2,
// gradients dlogits = softmax*(1 + 2z*lse) - onehot (fused_ce.py:80-84),
// dx = dlogits W, dW = dlogits^T x, both scaled by grad_output.
//
// Everything runs on one bf16 MFMA GEMM, C[m][n] = sum_k A[m][k] B[n][k]
// (both operands K-contiguous, "NT"), with four epilogues.  gemm_nt_dma takes
// K in whole 64-element slices: LDS-DMA rings of swizzled slices, 256 x 128
// tiles on 8 waves for the backward products and 256 x 256 tiles for the
// forward; gemm_nt (128 x 128 x 64, four waves of 64 x 64, register-staged)
// handles any other K.  Epilogues:
//   kLse      A = W, B = x: C = logits^T, lane <-> token.  Per token, a
//             (max, sum exp) partial over the tile's vocab rows and the
//             target logit; the [tokens x vocab] tile is discarded, or also
//             written as logits^T [vocab][tokens] (the _logits entry
//             points), from which dlogits_stored later forms dlogits with a
//             memory-bound pass instead of the kDlogits product.  With
//             round_bf16 the logits are rounded to bf16 before any use (and
//             stored as bf16), as the reference's bf16 x @ W^T product is.
//   kDlogits  same product over one vocab chunk; writes dlogits (scaled by the
//             device-resident grad_output) as dL [tokens][chunk] and dL^T.
//   kAccum    dx += dL W_chunk (fp32 accumulator; the last chunk writes x's dtype).
//   kStore    dW_chunk = dL^T x (written in W's dtype, or added to an fp32 dW).
// A small kernel merges the forward partials into lse / per-row loss, and a
// single workgroup sums the rows in a fixed order (deterministic scalar).
#include <math.h>

#include "common.hpp"
#include "lds_dma.hpp"

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
  void *lgt;               // kLse: optional logits^T [V][ldlg] (vocab-major), in
  int64_t ldlg;            //   bf16 when round_bf16 is set, else fp32
  int round_bf16;          // kLse / kDlogits: logits rounded to bf16 before use
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

// ---------------------------------------------------------------- DMA GEMM
// gemm_nt_dma: the product for K-slices that are whole multiples of 64, on
// tiles of WM x WN waves, each wave 32*IM x 32*JN (IM x JN MFMA blocks).  The
// A and B K-slices arrive by LDS DMA (16-byte buffer loads, rows past M / N
// read as zero) in the swizzled 128-byte-row layout of SwzTile<64>
// (conflict-free ds_read_b128 fragments, no padding), through a ring of
// STAGES slices: the slices STAGES-1 steps ahead are in flight while one is
// computed, with a single barrier per slice.  Workgroup i runs on XCD i % 8;
// each XCD takes a contiguous range of tiles in groups of kGroupM tile rows,
// so the workgroups resident on one XCD share A and B panels in its L2.
// gemm_nt (below) is the register-staged kernel for every other shape.
constexpr int kGroupM = 8;

__device__ __forceinline__ void tile_of(int id, int ntm, int ntn, int &tm, int &tn) {
  const int total = ntm * ntn;
  if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
  const int group = id / (kGroupM * ntn), first = group * kGroupM;
  const int rows = min(kGroupM, ntm - first);
  const int local = id - group * kGroupM * ntn;
  tm = first + local % rows;
  tn = local / rows;
}

// Epilogue of a finished tile (both kernels), WM x WN waves of 64*WM*WN
// threads: acc[i][j] of wave (wm, wn) = (wave / WN, wave % WN) holds rows
// m0 + 32*IM*wm + 32i + 8(r/4) + 4hh + r%4 and column n0 + 32*JN*wn + 32j + l32.
// kDlogits stages its bf16 rows (vocab-major, pitch BN + 8) in `stage`, one
// wave row (32*IM rows) at a time, so both dlogits layouts leave as 16-byte
// stores; the caller has finished every read of `stage` as an operand buffer.
template <int MODE, int WM, int WN, int IM, int JN>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs &g, f32x16_t (&acc)[IM][JN], int tm,
                                              int m0, int n0, bf16_t *stage,
                                              float (*red_m)[32 * JN * WN],
                                              float (*red_s)[32 * JN * WN],
                                              bool preloaded = false) {
  constexpr int NT = 64 * WM * WN, BNT = 32 * JN * WN, WR = 32 * IM, WC = 32 * JN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hh = lane >> 5, l32 = lane & 31;
  const int wm = wave / WN, wn = wave % WN;
  if constexpr (MODE == kLse || MODE == kDlogits) {
    if (g.round_bf16) {
#pragma unroll
      for (int i = 0; i < IM; ++i)
#pragma unroll
        for (int j = 0; j < JN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] = (float)(bf16_t)acc[i][j][r];
    }
  }
  if constexpr (MODE == kLse) {
    static_assert(NT >= BNT, "one thread per token column");
    if (g.lgt && g.round_bf16) {
      // bf16 logits^T, staged in LDS one 32-row accumulator block of one wave
      // row at a time (32 x BNT, pitch BNT + 8), so the rows leave as 16-byte
      // stores (columns past N land in the row padding, ldlg >= round8(N)).
      constexpr int TPS = BNT + 8, CPR = BNT / 8;
#pragma unroll
      for (int pass = 0; pass < WM * IM; ++pass) {
        const int pw = pass / IM, pi = pass % IM;
        __syncthreads();  // the staging rows are free
        if (wm == pw) {
#pragma unroll
          for (int j = 0; j < JN; ++j) {
            const int nl = WC * wn + 32 * j + l32;
#pragma unroll
            for (int r = 0; r < 16; ++r)
              stage[(8 * (r >> 2) + 4 * hh + (r & 3)) * TPS + nl] = (bf16_t)acc[pi][j][r];
          }
        }
        __syncthreads();
        const int mb = m0 + WR * pw + 32 * pi;
        for (int c = tid; c < 32 * CPR; c += NT) {
          const int ml = c / CPR, n = n0 + (c % CPR) * 8;
          if (mb + ml < g.M && n < g.N)
            *reinterpret_cast<u32x4 *>(static_cast<bf16_t *>(g.lgt) +
                                       (int64_t)(g.v0 + mb + ml) * g.ldlg + n) =
                *reinterpret_cast<const u32x4 *>(&stage[ml * TPS + (c % CPR) * 8]);
        }
      }
    } else if (g.lgt) {
      // fp32 logits^T: for each accumulator register, the 32 lanes of a
      // half-wave hold 32 consecutive tokens of one vocab row (128-byte runs).
#pragma unroll
      for (int j = 0; j < JN; ++j) {
        const int n = n0 + WC * wn + 32 * j + l32;
        if (n >= g.N) continue;
#pragma unroll
        for (int i = 0; i < IM; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = m0 + WR * wm + 32 * i + 8 * (r >> 2) + 4 * hh + (r & 3);
            if (m >= g.M) continue;
            static_cast<float *>(g.lgt)[(int64_t)(g.v0 + m) * g.ldlg + n] = acc[i][j][r];
          }
      }
    }
#pragma unroll
    for (int j = 0; j < JN; ++j) {
      const int nl = WC * wn + 32 * j + l32;
      const int n = n0 + nl;
      const bool nvalid = n < g.N;
      const int64_t t = nvalid ? g.targets[n] : g.ignore_index;
      const bool valid = nvalid && t != g.ignore_index;
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < IM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + WR * wm + 32 * i + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (m < g.M) {
            mx = fmaxf(mx, acc[i][j][r]);
            if (valid && (int64_t)(g.v0 + m) == t) g.tgt[n] = acc[i][j][r];
          }
        }
      mx *= kLog2e;
      float sm = 0.f;
#pragma unroll
      for (int i = 0; i < IM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + WR * wm + 32 * i + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (m < g.M) sm += fast_exp2(acc[i][j][r] * kLog2e - mx);
        }
      const float mo = __shfl_xor(mx, 32), so = __shfl_xor(sm, 32);
      const float mn = fmaxf(mx, mo);
      if (mn != -INFINITY) sm = sm * fast_exp2(mx - mn) + so * fast_exp2(mo - mn);
      if (hh == 0) {
        red_m[wm][nl] = mn;
        red_s[wm][nl] = sm;
      }
    }
    __syncthreads();
    if (tid < BNT) {
      const int n = n0 + tid;
      float m1 = red_m[0][tid], s1 = red_s[0][tid];
#pragma unroll
      for (int w = 1; w < WM; ++w) {
        const float m2 = red_m[w][tid], s2 = red_s[w][tid];
        const float mn = fmaxf(m1, m2);
        if (mn != -INFINITY) s1 = s1 * fast_exp2(m1 - mn) + s2 * fast_exp2(m2 - mn);
        m1 = mn;
      }
      if (n < g.N) {
        g.part_m[(int64_t)tm * g.N + n] = m1;
        g.part_s[(int64_t)tm * g.N + n] = s1;
      }
    }
  } else if constexpr (MODE == kDlogits) {
    static_assert(BNT == 128, "dlogits staging assumes 128 tokens per tile");
    static_assert((WR * 16) % NT == 0, "staging rows split evenly over the threads");
    constexpr int TPS = BNT + 8;  // staging row pitch (elements)
    constexpr int TG = NT / BNT;  // token-row groups per store sweep
    float lse2[JN], scale[JN], one[JN];
    int64_t tj[JN];
#pragma unroll
    for (int j = 0; j < JN; ++j) {
      const int n = n0 + WC * wn + 32 * j + l32;
      const bool nvalid = n < g.N;
      tj[j] = nvalid ? g.targets[n] : g.ignore_index;
      const bool valid = nvalid && tj[j] != g.ignore_index;
      const float lse = nvalid ? g.lse[n] : 0.f;
      lse2[j] = lse * kLog2e;
      scale[j] = valid ? (*g.grad_out) * (1.0f + 2.0f * g.z * lse) : 0.f;
      one[j] = valid ? (*g.grad_out) : 0.f;
    }
    for (int pass = 0; pass < WM; ++pass) {
      __syncthreads();  // the staging rows are free
      if (wm == pass) {
#pragma unroll
        for (int j = 0; j < JN; ++j) {
          const int nl = WC * wn + 32 * j + l32;
          const bool nvalid = n0 + nl < g.N;
#pragma unroll
          for (int i = 0; i < IM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int ml = 32 * i + 8 * (r >> 2) + 4 * hh + (r & 3);
              const int m = m0 + WR * pass + ml;
              float gv = fast_exp2(acc[i][j][r] * kLog2e - lse2[j]) * scale[j];
              if ((int64_t)(g.v0 + m) == tj[j]) gv -= one[j];
              stage[ml * TPS + nl] = (bf16_t)(m < g.M && nvalid ? gv : 0.f);
            }
        }
      }
      __syncthreads();
      const int mb = m0 + WR * pass;
      // dL^T [vocab][tokens]: 16 threads per 256-byte staging row.
#pragma unroll
      for (int k = 0; k < WR * 16 / NT; ++k) {
        const int c = tid + NT * k;
        const int ml = c >> 4, n8 = (c & 15) * 8;
        if (mb + ml < g.M && n0 + n8 < g.N)
          *reinterpret_cast<u32x4 *>(g.dlt + (int64_t)(mb + ml) * g.ldlt + n0 + n8) =
              *reinterpret_cast<const u32x4 *>(&stage[ml * TPS + n8]);
      }
      // dL [tokens][vocab]: lane <-> token, eight vocab rows per 16-byte store.
#pragma unroll
      for (int k = 0; k < WR * 16 / NT; ++k) {
        const int nl = tid & (BNT - 1), m8 = 8 * ((tid / BNT) + TG * k);
        if (n0 + nl < g.N && mb + m8 < g.M) {
          bf16x8_t v;
#pragma unroll
          for (int x = 0; x < 8; ++x) v[x] = stage[(m8 + x) * TPS + nl];
          *reinterpret_cast<bf16x8_t *>(g.dl + (int64_t)(n0 + nl) * g.ldl + mb + m8) = v;
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < IM; ++i)
#pragma unroll
      for (int j = 0; j < JN; ++j) {
        const int n = n0 + WC * wn + 32 * j + l32;
        if (n >= g.N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + WR * wm + 32 * i + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (m >= g.M) continue;
          float v = acc[i][j][r];
          if constexpr (MODE == kAccum) {
            if (g.part) {
              g.part[((int64_t)blockIdx.y * g.M + m) * g.N + n] = v;
              continue;
            }
            float *p = g.acc + (int64_t)m * g.ldc + n;
            if (!g.first && !preloaded) v += *p;
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

// Tile shape of one DMA-kernel instantiation: WM x WN waves of 32*IM x 32*JN
// outputs, K slices of KW elements (64 or 32: 128- or 64-byte LDS rows in
// the SwzTile<KW> swizzle), a ring of STAGES slices.
template <int WM_, int WN_, int IM_, int JN_, int STAGES_, int KW_ = 64>
struct DmaShape {
  static constexpr int WM = WM_, WN = WN_, IM = IM_, JN = JN_, STAGES = STAGES_, KW = KW_;
  static constexpr int NT = 64 * WM * WN, BMT = 32 * IM * WM, BNT = 32 * JN * WN;
};

template <int MODE, class SH>
__global__ __launch_bounds__(SH::NT) void gemm_nt_dma(GemmArgs g) {
  constexpr int WM = SH::WM, WN = SH::WN, IM = SH::IM, JN = SH::JN, STAGES = SH::STAGES;
  constexpr int KW = SH::KW, KB = 2 * KW, KS = KW / 16;  // slice width, row bytes, K steps
  constexpr int NT = SH::NT, BMT = SH::BMT, BNT = SH::BNT, W = NT / 64;
  constexpr int WR = 32 * IM, WC = 32 * JN;
  constexpr int AB = BMT * KB, SB = AB + BNT * KB;  // bytes of one stage (A then B)
  constexpr int NA = AB / (16 * NT), NB = BNT * KB / (16 * NT);  // DMAs per thread per stage
  constexpr int RB32 = 32 * KB;  // bytes of 32 rows: the offset between fragment row blocks
  static_assert(KW == 64 || KW == 32, "slice width");
  static_assert(NA * 16 * NT == AB && NB * 16 * NT == BNT * KB, "stage / thread mismatch");
  static_assert(STAGES >= 2 && STAGES <= 4, "ring of 2 to 4 slices");
  static_assert(MODE != kDlogits || WR * (BNT + 8) * 2 <= SB, "dlogits staging must fit a stage");
  static_assert(MODE != kLse || 32 * (BNT + 8) * 2 <= SB, "logits staging must fit a stage");
  // Stages are separate LDS objects, so the compiler does not wait for the
  // DMA into one before reading another.
  __shared__ __align__(16) char st0[SB], st1[SB], st2[STAGES > 2 ? SB : 16],
      st3[STAGES > 3 ? SB : 16];
  __shared__ float red_m[MODE == kLse ? WM : 1][BNT], red_s[MODE == kLse ? WM : 1][BNT];
  auto slot = [&](auto Ic) -> char * {
    constexpr int I = decltype(Ic)::value % STAGES;
    if constexpr (I == 0) return st0; else if constexpr (I == 1) return st1;
    else if constexpr (I == 2) return st2; else return st3;
  };
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hh = lane >> 5, l32 = lane & 31;
  const int wm = wave / WN, wn = wave % WN;
  const int ntm = (g.M + BMT - 1) / BMT, ntn = (g.N + BNT - 1) / BNT;
  int tm, tn;
  tile_of((int)blockIdx.x, ntm, ntn, tm, tn);
  const int m0 = tm * BMT, n0 = tn * BNT;
  const int kb = MODE == kAccum && g.part ? blockIdx.y * g.k_per_split : 0;
  const int ke = MODE == kAccum && g.part ? min(g.K, kb + g.k_per_split) : g.K;
  const int nk = (ke - kb) / KW;  // >= 1, checked by the host

  // DMA: chunk p of a stage <- row r, 16-byte chunk c of the K-slice.
  uint32_t aoff[NA], boff[NB];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    int r, c;
    SwzTile<KW>::at((i * W + wave) * 64 + lane, r, c);
    aoff[i] = (uint32_t)((r * g.lda + c * 8) * 2);
  }
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    int r, c;
    SwzTile<KW>::at((i * W + wave) * 64 + lane, r, c);
    boff[i] = (uint32_t)((r * g.ldb + c * 8) * 2);
  }
  const char *abase = reinterpret_cast<const char *>(g.A + (int64_t)m0 * g.lda + kb);
  const char *bbase = reinterpret_cast<const char *>(g.B + (int64_t)n0 * g.ldb + kb);
  // Valid bytes from the slice-0 base: through row M-1 (N-1), column ke.
  const int64_t alim = ((int64_t)(g.M - 1 - m0) * g.lda + (ke - kb)) * 2;
  const int64_t blim = ((int64_t)(g.N - 1 - n0) * g.ldb + (ke - kb)) * 2;
  // Slices past the last reload the last one into a slot nobody reads again,
  // so every step waits for the same DMA count.
  auto dma = [&](int t, char *dst) {
    const int64_t ko = (int64_t)(t < nk ? t : nk - 1) * KB;
#pragma unroll
    for (int i = 0; i < NA; ++i) dma16(abase + ko, alim - ko, aoff[i], dst + (i * W + wave) * 1024);
#pragma unroll
    for (int i = 0; i < NB; ++i)
      dma16(bbase + ko, blim - ko, boff[i], dst + AB + (i * W + wave) * 1024);
  };
  // Fragment offsets: rows WR*wm + 32i + l32 of A, WC*wn + 32j + l32 of B,
  // 16-byte chunk 2ks + hh.  The swizzle depends on the row only through
  // l32 (the row offsets are whole multiples of the swizzle period), so row
  // blocks differ by 32 rows.
  int aof[KS], bof[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    aof[ks] = SwzTile<KW>::off(WR * wm + l32, 16 * ks + 8 * hh);
    bof[ks] = AB + SwzTile<KW>::off(WC * wn + l32, 16 * ks + 8 * hh);
  }

  // kAccum after the first vocab chunk (no split-K): the MFMAs accumulate on
  // top of the fp32 sums of the earlier chunks, loaded here while the first
  // K slices' DMA is in flight, so the epilogue only stores (a read-modify-
  // write after the K loop left the matrix cores idle at one workgroup per CU).
  const bool preload = MODE == kAccum && !g.first && !g.part;
  f32x16_t acc[IM][JN];
#pragma unroll
  for (int i = 0; i < IM; ++i)
#pragma unroll
    for (int j = 0; j < JN; ++j) acc[i][j] = zero16();
  auto preload_acc = [&]() {
#pragma unroll
    for (int i = 0; i < IM; ++i)
#pragma unroll
      for (int j = 0; j < JN; ++j) {
        const int n = n0 + WC * wn + 32 * j + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + WR * wm + 32 * i + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (m < g.M && n < g.N) acc[i][j][r] = g.acc[(int64_t)m * g.ldc + n];
        }
      }
  };

  // Fragments are double-buffered across the slice's K steps: step ks+1's
  // LDS reads are in flight while step ks's MFMAs issue.
  auto compute = [&](const char *sb) {
    bf16x8_t a[2][IM], b[2][JN];
    auto load = [&](int ks, int buf) {
#pragma unroll
      for (int i = 0; i < IM; ++i)
        a[buf][i] = *reinterpret_cast<const bf16x8_t *>(sb + aof[ks] + RB32 * i);
#pragma unroll
      for (int j = 0; j < JN; ++j)
        b[buf][j] = *reinterpret_cast<const bf16x8_t *>(sb + bof[ks] + RB32 * j);
    };
    load(0, 0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      // sched_barrier keeps the scheduler from sinking the reads back
      // behind the MFMAs (it would reuse one fragment buffer otherwise).
      __builtin_amdgcn_sched_barrier(0);
      if (ks + 1 < KS) load(ks + 1, (ks + 1) & 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < IM; ++i)
#pragma unroll
        for (int j = 0; j < JN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[ks & 1][i], b[ks & 1][j],
                                                               acc[i][j], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // One step: slice kt (in slot kt % STAGES) has landed for this thread, the
  // barrier makes it visible and frees slot (kt - 1) % STAGES, which takes
  // slice kt + STAGES - 1.
  auto step = [&](int kt, auto Ic) {
    constexpr int I = decltype(Ic)::value;
    wait_vmcnt<(STAGES - 2) * (NA + NB)>();
    block_sync_nofence();
    dma(kt + STAGES - 1, slot(std::integral_constant<int, I + STAGES - 1>()));
    compute(slot(Ic));
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  dma(0, st0);
  if constexpr (STAGES > 2) dma(1, st1);
  if constexpr (STAGES > 3) dma(2, st2);
  if constexpr (MODE == kAccum)
    if (preload) preload_acc();
  int kt = 0;
  for (; kt + STAGES <= nk; kt += STAGES) {
    step(kt, I0());
    step(kt + 1, I1());
    if constexpr (STAGES > 2) step(kt + 2, I2());
    if constexpr (STAGES > 3) step(kt + 3, I3());
  }
  if (kt < nk) step(kt, I0());
  if constexpr (STAGES > 2)
    if (kt + 1 < nk) step(kt + 1, I1());
  if constexpr (STAGES > 3)
    if (kt + 2 < nk) step(kt + 2, I2());
  wait_vmcnt<0>();
  __syncthreads();  // every wave is done with the stages (kDlogits / kLse stage in st0)
  gemm_epilogue<MODE, WM, WN, IM, JN>(g, acc, tm, m0, n0, reinterpret_cast<bf16_t *>(st0), red_m,
                                      red_s, preload);
}

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

  gemm_epilogue<MODE, 2, 2, 2, 2>(g, acc, tm, m0, n0, smem, red_m, red_s);
}

// out (+)= sum of the split-K partials (the kAccum epilogue, applied after a
// split-K GEMM): fp32 accumulator in between chunks, out dtype at the end.
// dlogits of one vocab chunk from the forward's stored bf16 logits^T (the
// kDlogits product without recomputing the logits):
//   dL = (exp(logit - lse) (1 + 2z lse) - onehot) * grad_out,
// written as dL^T [vc][ldlt] (the logits' own layout) and dL [n][ldl]
// (transposed through LDS).  Tile: 128 vocab rows x 128 tokens (256-byte row
// segments), 256 threads; thread t handles tokens 8 (t % 16) .. +7 of rows
// t / 16 + 16 k, with 16-byte loads and stores (non-temporal ones measured
// 3x slower here).  Rows and tokens past the chunk / n are zeros.
constexpr int kDlRows = 128, kDlTokens = 128;  // dlogits_stored tile (vocab rows x tokens)
static_assert(256 % (kDlTokens / 8) == 0 && kDlRows % (256 / (kDlTokens / 8)) == 0 &&
                  256 % kDlTokens == 0 && (kDlRows / (256 / kDlTokens)) % 8 == 0,
              "dlogits_stored tile");

struct DlArgs {
  const void *lg;  // logits^T [V][ldlg] (bf16 or fp32), rows v0 .. v0 + vc - 1 used
  int64_t ldlg;
  int v0, vc, n;
  const int64_t *targets;
  int64_t ignore_index;
  float z;
  const float *lse;       // [n] natural-log lse
  const float *grad_out;  // device scalar
  bf16_t *dl, *dlt;
  int64_t ldl, ldlt;
};

template <typename T>
__global__ __launch_bounds__(256) void dlogits_stored(DlArgs a) {
  constexpr int TM = kDlRows, TN = kDlTokens, TP = TN + 8;  // staging pitch (elements)
  constexpr int GN = TN / 8, RS = 256 / GN;  // token groups of 8; rows per pass
  __shared__ __align__(16) bf16_t st[TM * TP];
  const int tid = threadIdx.x;
  const int c8 = (tid % GN) * 8, r0 = tid / GN;
  const int m0 = (int)blockIdx.x * TM, n0 = (int)blockIdx.y * TN;
  const int n = n0 + c8;
  const float g = *a.grad_out;
  float lse2[8], scale[8], one[8];
  int64_t tg[8];
#pragma unroll
  for (int x = 0; x < 8; ++x) {
    const int nn = n + x;
    const bool nvalid = nn < a.n;
    tg[x] = nvalid ? a.targets[nn] : a.ignore_index;
    const bool valid = nvalid && tg[x] != a.ignore_index;
    const float lse = nvalid ? a.lse[nn] : 0.f;
    lse2[x] = lse * kLog2e;
    scale[x] = valid ? g * (1.0f + 2.0f * a.z * lse) : 0.f;
    one[x] = valid ? g : 0.f;
  }
  // Every row's logits are loaded before the first store: a store to dL^T
  // between two loads would keep the compiler from issuing the next load
  // (it cannot tell the buffers apart), one memory latency per row.
  float lv[TM / RS][8];
  if (m0 + TM <= a.vc && n0 + TN <= a.n) {  // whole tile in range (uniform)
    constexpr int NQ = sizeof(T) * 8 / 16;     // 16-byte vectors per row segment
    u32x4 raw[TM / RS][NQ];
#pragma unroll
    for (int rr = 0; rr < TM / RS; ++rr) {
      const T *src = static_cast<const T *>(a.lg) + (int64_t)(a.v0 + m0 + r0 + RS * rr) * a.ldlg + n;
#pragma unroll
      for (int q = 0; q < NQ; ++q) raw[rr][q] = reinterpret_cast<const u32x4 *>(src)[q];
    }
#pragma unroll
    for (int rr = 0; rr < TM / RS; ++rr) {
      const T *e = reinterpret_cast<const T *>(&raw[rr][0]);
#pragma unroll
      for (int x = 0; x < 8; ++x) lv[rr][x] = (float)e[x];
    }
  } else {
#pragma unroll
  for (int rr = 0; rr < TM / RS; ++rr) {
    const int m = m0 + r0 + RS * rr;
#pragma unroll
    for (int x = 0; x < 8; ++x) lv[rr][x] = 0.f;
    if (m < a.vc && n < a.n) {
      const T *src = static_cast<const T *>(a.lg) + (int64_t)(a.v0 + m) * a.ldlg + n;
      if (n + 8 <= a.n) {
        if constexpr (sizeof(T) == 2) {
          load16(src, lv[rr]);
        } else {
          float lo[4], hi[4];
          load16(src, lo);
          load16(src + 4, hi);
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            lv[rr][x] = lo[x];
            lv[rr][4 + x] = hi[x];
          }
        }
      } else {
#pragma unroll
        for (int x = 0; x < 8; ++x) lv[rr][x] = n + x < a.n ? (float)src[x] : 0.f;
      }
    }
  }
  }
#pragma unroll
  for (int rr = 0; rr < TM / RS; ++rr) {
    const int ml = r0 + RS * rr, m = m0 + ml;
    bf16x8_t o;
    if (m < a.vc && n < a.n) {
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        float gv = fast_exp2(lv[rr][x] * kLog2e - lse2[x]) * scale[x];
        if ((int64_t)(a.v0 + m) == tg[x]) gv -= one[x];
        o[x] = (bf16_t)(n + x < a.n ? gv : 0.f);
      }
    } else {
#pragma unroll
      for (int x = 0; x < 8; ++x) o[x] = (bf16_t)0.0f;
    }
    if (m < a.vc && n < a.ldlt) *reinterpret_cast<bf16x8_t *>(a.dlt + (int64_t)m * a.ldlt + n) = o;
    *reinterpret_cast<bf16x8_t *>(&st[ml * TP + c8]) = o;
  }
  __syncthreads();
  // dL: token row nl, TM / 2 vocab columns from mc (16-byte stores).
  constexpr int TPR = 256 / TN, MC = TM / TPR;  // threads per token row, columns each
  const int nl = tid / TPR, mc = (tid % TPR) * MC, nn = n0 + nl;
  if (nn < a.n) {
#pragma unroll
    for (int h = 0; h < MC / 8; ++h) {
      const int m = m0 + mc + 8 * h;
      if (m < a.vc) {
        bf16x8_t v;
#pragma unroll
        for (int x = 0; x < 8; ++x) v[x] = st[(mc + 8 * h + x) * TP + nl];
        *reinterpret_cast<bf16x8_t *>(a.dl + (int64_t)nn * a.ldl + m) = v;
      }
    }
  }
}

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

// Tile shape of the DMA kernel: 256 x 128 on 8 waves (two per SIMD), a
// three-slice ring of 48 KiB slices.  Smaller tiles need more bytes per flop
// and a 2-slice ring does not cover the operand latency (measured slower).
using RowShape = DmaShape<4, 2, 2, 2, 3>;
// 256 x 256 tiles on 8 waves of 128 x 64 (6 fragment reads per 8 MFMAs
// instead of 4 per 4, half the operand bytes per flop), 32-wide K slices in
// a four-slice ring of 32 KiB.  Used for the forward (lse) product when the
// grid still has >= 1024 tiles (four per CU): cfg4 16.1 -> 15.6 ms.  The
// backward products measured slower on it (dx and dW 51.8 -> 52.8 ms for
// the chunk loop), and dlogits' staging takes 128 tokens, so they keep
// RowShape.
using WideShape = DmaShape<2, 4, 4, 2, 4, 32>;
template <class SH> unsigned dma_tiles(int m, int n) {
  return (unsigned)(((m + SH::BMT - 1) / SH::BMT) * ((n + SH::BNT - 1) / SH::BNT));
}
// The DMA kernel takes K-slices of whole 64-element blocks (operands are
// already 16-byte aligned with row strides % 8 == 0).
bool dma_ok(int64_t k) { return k > 0 && k % 64 == 0; }
bool wide_ok(int64_t m, int64_t n, int64_t k) {
  return dma_ok(k) && dma_tiles<WideShape>((int)m, (int)n) >= 1024;
}

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

namespace {
int lmhead_fwd(const void *x, int64_t ldx, const void *w, int64_t ldw, int64_t n, int64_t v,
               int64_t d, const int64_t *targets, int64_t ignore_index, float z_loss_coeff,
               float *loss_rows, float *lse, float *loss_sum, void *workspace, bool round_bf16,
               void *logits, int64_t ldlg, void *stream) {
  using namespace pb;
  using namespace pb::ce;
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
  const bool dma = dma_ok(d), wide = wide_ok(v, n, d);
  const int bm = wide ? WideShape::BMT : dma ? RowShape::BMT : BM;  // lse partials per token
  const int nmt = (int)((v + bm - 1) / bm);
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
  g.lgt = logits;
  g.ldlg = ldlg;
  g.round_bf16 = round_bf16;
  if (wide)
    hipLaunchKernelGGL((gemm_nt_dma<kLse, WideShape>), dim3(dma_tiles<WideShape>(g.M, g.N)),
                       dim3(WideShape::NT), 0, st, g);
  else if (dma)
    hipLaunchKernelGGL((gemm_nt_dma<kLse, RowShape>), dim3(dma_tiles<RowShape>(g.M, g.N)),
                       dim3(RowShape::NT), 0, st, g);
  else
    hipLaunchKernelGGL(gemm_nt<kLse>, dim3(tiles(g.M, g.N)), dim3(256), 0, st, g);
  int rc = launch_status("pb_lmhead_ce_fwd(gemm)");
  if (rc) return rc;
  hipLaunchKernelGGL(lse_combine, dim3((unsigned)((n + 63) / 64)), dim3(1024), 0, st, g.part_m,
                     g.part_s, nmt, (int)n, g.tgt, targets, ignore_index, (int)v, z_loss_coeff, lse,
                     loss_rows);
  hipLaunchKernelGGL(sum_rows, dim3(1), dim3(1024), 0, st, loss_rows, (int)n, loss_sum);
  return launch_status("pb_lmhead_ce_fwd");
}
}  // namespace

extern "C" int pb_lmhead_ce_fwd(const void *x, int64_t ldx, const void *w, int64_t ldw,
                                int64_t n, int64_t v, int64_t d, const int64_t *targets,
                                int64_t ignore_index, float z_loss_coeff, float *loss_rows,
                                float *lse, float *loss_sum, void *workspace, void *stream) {
  pb::clear_error();
  return lmhead_fwd(x, ldx, w, ldw, n, v, d, targets, ignore_index, z_loss_coeff, loss_rows, lse,
                    loss_sum, workspace, false, nullptr, 0, stream);
}

extern "C" int pb_lmhead_ce_fwd_logits(const void *x, int64_t ldx, const void *w, int64_t ldw,
                                       int64_t n, int64_t v, int64_t d, const int64_t *targets,
                                       int64_t ignore_index, float z_loss_coeff, float *loss_rows,
                                       float *lse, float *loss_sum, void *workspace,
                                       int logits_dtype, void *logits, int64_t ldlg,
                                       void *stream) {
  pb::clear_error();
  PB_CHECK_ARG(logits_dtype == PB_BF16 || logits_dtype == PB_F32,
               "pb_lmhead_ce_fwd_logits: logits_dtype must be bf16 or fp32");
  PB_CHECK_ARG(logits == nullptr || (ldlg >= n && ldlg % 8 == 0 &&
                                     reinterpret_cast<uintptr_t>(logits) % 16 == 0),
               "pb_lmhead_ce_fwd_logits: logits must be 16-byte aligned with ldlg >= n, "
               "ldlg %% 8 == 0");
  return lmhead_fwd(x, ldx, w, ldw, n, v, d, targets, ignore_index, z_loss_coeff, loss_rows, lse,
                    loss_sum, workspace, logits_dtype == PB_BF16, logits, ldlg, stream);
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
  // Split the dx GEMM's K (vocab chunk) when its tile grid (counted in the
  // DMA kernel's 256 x 128 tiles, one workgroup per CU) cannot fill the
  // GPU: of 1..8 splits of at least kmin columns, the one whose grid takes the
  // least time as (rounds of 256 workgroups) x (K columns per split), fewer
  // splits on a tie.  E.g. 96 tiles: 8 splits = 3 full rounds of 4032
  // columns against 6 splits = 2.25 rounds (a quarter-full third round) of
  // 5376.
  const int64_t tiles = ((n + 255) / 256) * ((d + 127) / 128);
  constexpr int64_t kCus = 256, kmin = 1024;
  auto kps = [&](int64_t s) {
    return ((vchunk + s - 1) / s + pb::ce::BK - 1) / pb::ce::BK * pb::ce::BK;
  };
  int64_t splits = 1, best = (tiles + kCus - 1) / kCus * kps(1);
  for (int64_t s = 2; s <= 8 && vchunk / s >= kmin; ++s) {
    const int64_t cost = (tiles * s + kCus - 1) / kCus * kps(s);
    if (cost < best) {
      best = cost;
      splits = s;
    }
  }
  w.splits = (int)splits;
  w.k_per_split = (int)kps(splits);
  w.bytes = w.off_part + (splits > 1 ? al(splits * n * d * 4) : 0);
  return w;
}
}  // namespace

extern "C" int64_t pb_lmhead_ce_bwd_workspace_bytes(int64_t n, int64_t v, int64_t d,
                                                    int64_t vchunk) {
  if (n <= 0 || v <= 0 || d <= 0 || vchunk <= 0) return 0;
  return bwd_ws(n, v, d, vchunk).bytes;
}

namespace {
// dL [n][vc] (row stride ldl) and dL^T [vc][ldlt] of vocab rows v0 .. v0 + vc:
// from the stored logits^T when given, else by the recomputing GEMM.
int dlogits_chunk(const void *x, int64_t ldx, const void *w, int64_t ldw, int64_t n, int64_t v,
                  int64_t d, const int64_t *targets, int64_t ignore_index, float z_loss_coeff,
                  const float *lse, const float *grad_out, int64_t v0, int vc, pb::bf16_t *dl,
                  int64_t ldl, pb::bf16_t *dlt, int64_t ldlt, bool round_bf16, const void *logits,
                  int64_t ldlg, hipStream_t st) {
  using namespace pb;
  using namespace pb::ce;
  if (logits) {
    DlArgs da = {};
    da.lg = static_cast<const bf16_t *>(logits);
    da.ldlg = ldlg;
    da.v0 = (int)v0; da.vc = vc; da.n = (int)n;
    da.targets = targets;
    da.ignore_index = ignore_index;
    da.z = z_loss_coeff;
    da.lse = lse;
    da.grad_out = grad_out;
    da.dl = dl; da.dlt = dlt;
    da.ldl = ldl; da.ldlt = ldlt;
    const dim3 grid((unsigned)((vc + kDlRows - 1) / kDlRows),
                    (unsigned)((n + kDlTokens - 1) / kDlTokens));
    if (round_bf16)
      hipLaunchKernelGGL(dlogits_stored<bf16_t>, grid, dim3(256), 0, st, da);
    else
      hipLaunchKernelGGL(dlogits_stored<float>, grid, dim3(256), 0, st, da);
    return launch_status("pb_lmhead_ce(dlogits)");
  }
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
  g.round_bf16 = round_bf16;
  if (dma_ok(d))
    hipLaunchKernelGGL((gemm_nt_dma<kDlogits, RowShape>), dim3(dma_tiles<RowShape>(g.M, g.N)),
                       dim3(RowShape::NT), 0, st, g);
  else
    hipLaunchKernelGGL(gemm_nt<kDlogits>, dim3(tiles(g.M, g.N)), dim3(256), 0, st, g);
  return launch_status("pb_lmhead_ce(dlogits)");
}

int lmhead_bwd(const void *x, int64_t ldx, const void *w, int64_t ldw, const void *xt,
               int64_t ldxt, const void *wt, int64_t ldwt, int64_t n, int64_t v, int64_t d,
               const int64_t *targets, int64_t ignore_index, float z_loss_coeff,
               const float *lse, const float *grad_out, int64_t vchunk, void *workspace,
               void *dx, int dx_dtype, int64_t lddx, void *dw, int dw_dtype, int64_t lddw,
               int dw_accumulate, bool round_bf16, const void *logits, int64_t ldlg,
               void *stream) {
  using namespace pb;
  using namespace pb::ce;
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
    // 1) dlogits for vocab rows [v0, v0 + vc): dL [n][vc], dL^T [vc][n] --
    // from the stored logits, or by recomputing them.
    int rc = dlogits_chunk(x, ldx, w, ldw, n, v, d, targets, ignore_index, z_loss_coeff, lse,
                           grad_out, v0, vc, dl, ldl, dlt, ldlt, round_bf16, logits, ldlg, st);
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
    if (dma_ok(vc))
      hipLaunchKernelGGL((gemm_nt_dma<kAccum, RowShape>), dim3(dma_tiles<RowShape>(gx.M, gx.N), splits),
                         dim3(RowShape::NT), 0, st, gx);
    else
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
    if (dma_ok(n))
      hipLaunchKernelGGL((gemm_nt_dma<kStore, RowShape>), dim3(dma_tiles<RowShape>(gw.M, gw.N)),
                         dim3(RowShape::NT), 0, st, gw);
    else
      hipLaunchKernelGGL(gemm_nt<kStore>, dim3(tiles(gw.M, gw.N)), dim3(256), 0, st, gw);
    rc = launch_status("pb_lmhead_ce_bwd(dx/dw)");
    if (rc) return rc;
  }
  return PB_OK;
}
}  // namespace

extern "C" int pb_lmhead_ce_bwd(const void *x, int64_t ldx, const void *w, int64_t ldw,
                                const void *xt, int64_t ldxt, const void *wt, int64_t ldwt,
                                int64_t n, int64_t v, int64_t d, const int64_t *targets,
                                int64_t ignore_index, float z_loss_coeff, const float *lse,
                                const float *grad_out, int64_t vchunk, void *workspace, void *dx,
                                int dx_dtype, int64_t lddx, void *dw, int dw_dtype, int64_t lddw,
                                int dw_accumulate, void *stream) {
  pb::clear_error();
  return lmhead_bwd(x, ldx, w, ldw, xt, ldxt, wt, ldwt, n, v, d, targets, ignore_index,
                    z_loss_coeff, lse, grad_out, vchunk, workspace, dx, dx_dtype, lddx, dw,
                    dw_dtype, lddw, dw_accumulate, false, nullptr, 0, stream);
}

extern "C" int pb_lmhead_ce_bwd_logits(const void *x, int64_t ldx, const void *w, int64_t ldw,
                                       const void *xt, int64_t ldxt, const void *wt, int64_t ldwt,
                                       int64_t n, int64_t v, int64_t d, const int64_t *targets,
                                       int64_t ignore_index, float z_loss_coeff, const float *lse,
                                       const float *grad_out, int64_t vchunk, void *workspace,
                                       void *dx, int dx_dtype, int64_t lddx, void *dw,
                                       int dw_dtype, int64_t lddw, int dw_accumulate,
                                       int logits_dtype, const void *logits, int64_t ldlg,
                                       void *stream) {
  pb::clear_error();
  PB_CHECK_ARG(logits_dtype == PB_BF16 || logits_dtype == PB_F32,
               "pb_lmhead_ce_bwd_logits: logits_dtype must be bf16 or fp32");
  PB_CHECK_ARG(logits == nullptr || (ldlg >= n && ldlg % 8 == 0 &&
                                     reinterpret_cast<uintptr_t>(logits) % 16 == 0),
               "pb_lmhead_ce_bwd_logits: logits must be 16-byte aligned with ldlg >= n, "
               "ldlg %% 8 == 0");
  PB_CHECK_SUPPORTED(logits == nullptr || (n + pb::ce::kDlTokens - 1) / pb::ce::kDlTokens <= 65535,
                     "pb_lmhead_ce_bwd_logits: too many rows for stored logits");
  return lmhead_bwd(x, ldx, w, ldw, xt, ldxt, wt, ldwt, n, v, d, targets, ignore_index,
                    z_loss_coeff, lse, grad_out, vchunk, workspace, dx, dx_dtype, lddx, dw,
                    dw_dtype, lddw, dw_accumulate, logits_dtype == PB_BF16, logits, ldlg, stream);
}

extern "C" int pb_lmhead_ce_dlogits(const void *x, int64_t ldx, const void *w, int64_t ldw,
                                    int64_t n, int64_t v, int64_t d, const int64_t *targets,
                                    int64_t ignore_index, float z_loss_coeff, const float *lse,
                                    const float *grad_out, int64_t v0, int64_t vc, void *dl,
                                    int64_t ldl, void *dlt, int64_t ldlt, int logits_dtype,
                                    const void *logits, int64_t ldlg, void *stream) {
  using namespace pb;
  using namespace pb::ce;
  clear_error();
  PB_CHECK_ARG(n >= 1 && v >= 1 && d >= 1 && vc >= 1 && v0 >= 0 && v0 + vc <= v,
               "pb_lmhead_ce_dlogits: bad shape or chunk");
  PB_CHECK_SUPPORTED(n < (1LL << 31) && v < (1LL << 31) && d < (1LL << 31),
                     "pb_lmhead_ce_dlogits: too large");
  PB_CHECK_ARG(logits_dtype == PB_BF16 || logits_dtype == PB_F32,
               "pb_lmhead_ce_dlogits: logits_dtype must be bf16 or fp32");
  PB_CHECK_ARG(x && w && targets && lse && grad_out && dl && dlt,
               "pb_lmhead_ce_dlogits: null argument");
  PB_CHECK_ARG(k_aligned(x, ldx) && k_aligned(w, ldw) && d % 8 == 0 && k_aligned(dl, ldl) &&
                   k_aligned(dlt, ldlt) && ldl >= vc && ldlt >= n,
               "pb_lmhead_ce_dlogits: operands must be 16-byte aligned with row strides %% 8 == 0 "
               "(ldl >= vc, ldlt >= n)");
  PB_CHECK_ARG(logits == nullptr || (ldlg >= n && ldlg % 8 == 0 &&
                                     reinterpret_cast<uintptr_t>(logits) % 16 == 0),
               "pb_lmhead_ce_dlogits: logits must be 16-byte aligned with ldlg >= n, "
               "ldlg %% 8 == 0");
  PB_CHECK_SUPPORTED(logits == nullptr || (n + kDlTokens - 1) / kDlTokens <= 65535,
                     "pb_lmhead_ce_dlogits: too many rows for stored logits");
  return dlogits_chunk(x, ldx, w, ldw, n, v, d, targets, ignore_index, z_loss_coeff, lse,
                       grad_out, v0, (int)vc, static_cast<bf16_t *>(dl), ldl,
                       static_cast<bf16_t *>(dlt), ldlt, logits_dtype == PB_BF16, logits, ldlg,
                       as_stream(stream));
}
