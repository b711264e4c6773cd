/*
 * packbalance_amd.h -- C ABI of the MI355X (gfx950) kernels behind PackBalance's
 * training hot path: document-masked GQA attention, RMSNorm, SwiGLU and the
 * LM-head cross-entropy.
 *
 * Conventions shared by every entry point
 *   - Pointers are device pointers (HBM); sizes and strides are int64 element
 *     counts; the innermost dimension of every matrix has unit stride.
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream).
 *     Every entry point only enqueues work: no allocation, no host sync.
 *   - Return value: PB_OK, or a negative status; pb_last_error() returns a
 *     thread-local message describing the last failure on the calling thread.
 *   - Inputs are never written.  Workspaces are caller-owned.
 *
 * Each declaration names the reference function it replaces
 * (paths are relative to the DeKodez/packbalance source tree).
 */
#ifndef PACKBALANCE_AMD_H
#define PACKBALANCE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define PB_OK 0
#define PB_EINVAL (-1)       /* bad shape / argument   -> Python ValueError   */
#define PB_EUNSUPPORTED (-2) /* size/dtype not handled -> Python RuntimeError */
#define PB_EHIP (-3)         /* HIP launch error       -> Python RuntimeError */

/* ---- element types ------------------------------------------------------ */
#define PB_F32 0
#define PB_BF16 1
#define PB_F16 2

/* Message for the last failing call on this thread ("" if none). */
const char *pb_last_error(void);

/* ABI version of this library; bumped whenever a signature changes. */
int pb_abi_version(void);

/* ---- RMSNorm ------------------------------------------------------------
 * Replaces packbalance/kernels/rmsnorm.py:29-48 (_rmsnorm_fwd) and the
 * forward of _RMSNorm (rmsnorm.py:77-99).
 *   rstd[r] = 1/sqrt(mean_c(x[r,c]^2) + eps)    (fp32)
 *   y[r,c]  = x[r,c] * rstd[r] * w[c]            (fp32 math, stored as x_dtype)
 * x_dtype, w_dtype in {PB_F32, PB_BF16, PB_F16}; y has x_dtype.
 * n <= 65536 (rmsnorm.py:81-82 limit), else PB_EUNSUPPORTED.            */
int pb_rmsnorm_fwd(const void *x, int64_t x_row_stride, int x_dtype,
                   const void *w, int w_dtype, void *y, int64_t y_row_stride,
                   float *rstd, int64_t rows, int64_t n, float eps,
                   void *stream);

/* Bytes of fp32 workspace pb_rmsnorm_bwd needs for its dw partial sums. */
int64_t pb_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t n);

/* Replaces rmsnorm.py:51-72 (_rmsnorm_bwd) and the eager dw reduction of
 * _RMSNorm.backward (rmsnorm.py:117-118), fused:
 *   g = dy*w, xh = x*rstd, dx = rstd*(g - xh*mean_c(g*xh))   (stored as dy dtype = x_dtype)
 *   dw[c] = sum_r dy[r,c]*xh[r,c]   (fp32 accumulate, stored as w_dtype)
 * `workspace` holds pb_rmsnorm_bwd_workspace_bytes(rows, n) bytes.          */
int pb_rmsnorm_bwd(const void *dy, int64_t dy_row_stride, const void *x,
                   int64_t x_row_stride, int x_dtype, const void *w,
                   int w_dtype, const float *rstd, void *dx,
                   int64_t dx_row_stride, void *dw, void *workspace,
                   int64_t rows, int64_t n, void *stream);

/* No counterpart in the reference: pb_rmsnorm_bwd for callers that cannot
 * allocate (code under graph capture without a caller-held workspace, tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments and results
 * as pb_rmsnorm_bwd minus `workspace`: the dW partial rows live in a static
 * per-GPU device array of PB_RMSNORM_NOALLOC_SCRATCH_BYTES (held by every GPU
 * the library runs on until the process ends).  Calls needing more
 * (pb_rmsnorm_bwd_workspace_bytes(rows, n) > the limit) return
 * PB_EUNSUPPORTED; every rows count at n <= 8192 fits.  Every call on one GPU
 * shares the array: calls that overlap on one GPU (other streams or threads)
 * race.                                                                     */
#define PB_RMSNORM_NOALLOC_SCRATCH_BYTES (16 * 1024 * 1024)
int pb_rmsnorm_bwd_noalloc(const void *dy, int64_t dy_row_stride, const void *x,
                           int64_t x_row_stride, int x_dtype, const void *w,
                           int w_dtype, const float *rstd, void *dx,
                           int64_t dx_row_stride, void *dw, int64_t rows,
                           int64_t n, void *stream);

/* ---- SwiGLU -------------------------------------------------------------
 * Replaces packbalance/kernels/swiglu.py:23-31 (_swiglu_fwd):
 *   out = g*sigmoid(g)*u   over n contiguous elements (fp32 math).      */
int pb_swiglu_fwd(const void *gate, const void *up, void *out, int64_t n,
                  int dtype, void *stream);

/* Replaces swiglu.py:34-46 (_swiglu_bwd):
 *   dgate = dy*u*s*(1+g*(1-s)), dup = dy*g*s,  s = sigmoid(g).           */
int pb_swiglu_bwd(const void *gate, const void *up, const void *dy,
                  void *dgate, void *dup, int64_t n, int dtype, void *stream);

/* Row-strided forms of the two above (same math): every operand is a
 * [rows, cols] block with its own row stride (elements) and unit column
 * stride, so gate/up may be the two halves of one fused [rows, 2*cols]
 * projection and dgate/dup may be written back into one such buffer.
 * Replaces the same reference functions (swiglu.py:23-46), which reach
 * them through .contiguous() copies of non-contiguous gate/up.              */
int pb_swiglu_fwd_rows(const void *gate, int64_t gate_row_stride,
                       const void *up, int64_t up_row_stride, void *out,
                       int64_t out_row_stride, int64_t rows, int64_t cols,
                       int dtype, void *stream);
int pb_swiglu_bwd_rows(const void *gate, int64_t gate_row_stride,
                       const void *up, int64_t up_row_stride, const void *dy,
                       int64_t dy_row_stride, void *dgate,
                       int64_t dgate_row_stride, void *dup,
                       int64_t dup_row_stride, int64_t rows, int64_t cols,
                       int dtype, void *stream);

/* ---- Row cross-entropy over a materialised logits block ----------------
 * Replaces packbalance/kernels/fused_ce.py:31-89 (_ce_kernel) and
 * _ce_launch (fused_ce.py:91-118).  Per row r of logits[m, v] (any strides):
 *   lse = logsumexp_c logits[r,c]
 *   loss[r] = lse - logits[r,t] + z*lse^2,    0 when t == ignore_index
 *   dlogits[r,c] = softmax*(1+2z*lse) - [c==t], 0 rows for ignored targets
 * dlogits (same dtype and strides as logits) is written only if non-NULL;
 * lse_out (fp32 [m]) only if non-NULL.  targets are int64.  A target outside
 * [0, v) that is not ignore_index is never dereferenced: its row's loss is
 * NaN and its dlogits row carries no one-hot term.                          */
int pb_ce_rows(const void *logits, int64_t stride_m, int64_t stride_v,
               int dtype, const int64_t *targets, float *loss, float *lse_out,
               void *dlogits, int64_t m, int64_t v, int64_t ignore_index,
               float z_loss_coeff, void *stream);

/* pb_ce_rows with dlogits of its own dtype and strides (the same values,
 * rounded once to dl_dtype), e.g. fp32 logits from a GEMM with fp32 output
 * and the bf16 dlogits a gradient GEMM consumes, in one pass.  Extends
 * _ce_launch (fused_ce.py:91-118), whose dlogits is always
 * empty_like(logits).                                                       */
int pb_ce_rows_dl(const void *logits, int64_t stride_m, int64_t stride_v,
                  int dtype, const int64_t *targets, float *loss, float *lse_out,
                  void *dlogits, int64_t dl_stride_m, int64_t dl_stride_v,
                  int dl_dtype, int64_t m, int64_t v, int64_t ignore_index,
                  float z_loss_coeff, void *stream);

/* ---- Document block tables (FlexAttention BlockMask layout) -------------
 * Replaces packbalance/model/attention.py:25-54 (build_doc_block_mask) with
 * torch.nn.attention.flex_attention.create_block_mask's table semantics:
 * mask(q, kv) = doc[q] == doc[kv] && q >= kv, positions >= s are masked,
 * a block is FULL when all block*block entries are allowed, PARTIAL when
 * some are.  Index rows list the set blocks ascending, then the unset blocks
 * ascending (argsort(descending, stable)).
 *   doc_ids  int64 [b, s] (row stride doc_stride)
 *   outputs  int32, replicated over h heads, contiguous:
 *     kv_num, full_kv_num        [b, h, nq]
 *     kv_idx, full_kv_idx        [b, h, nq, nkv]
 *     q_num, full_q_num          [b, h, nkv]
 *     q_idx, full_q_idx          [b, h, nkv, nq]
 *   with nq = nkv = ceil(s / block).
 *   `class_ws` is a workspace of b*nq*nkv bytes (block class per tile).      */
int pb_doc_block_tables(const int64_t *doc_ids, int64_t doc_stride, int64_t b,
                        int64_t s, int64_t block, int64_t h, int32_t *kv_num,
                        int32_t *kv_idx, int32_t *full_kv_num,
                        int32_t *full_kv_idx, int32_t *q_num, int32_t *q_idx,
                        int32_t *full_q_num, int32_t *full_q_idx,
                        uint8_t *class_ws, void *stream);

/* ---- Document-masked GQA attention --------------------------------------
 * A [B, H, S, D] tensor view: element strides for b, h, s; D is unit-stride.
 * The model's q/k/v are .transpose(1, 2) views of [B, S, H, D] memory
 * (packbalance/model/llama.py:86-92), so any stride order is accepted.      */
typedef struct pb_bhsd {
  void *data;
  int64_t stride_b;
  int64_t stride_h;
  int64_t stride_s;
} pb_bhsd;

/* Launch configuration of the attention kernels for one problem shape (no
 * reference counterpart).  out[0..9] = forward query tile, forward KV tile,
 * dK/dV query tile, dK/dV KV tile, dQ query tile, dQ KV tile, pb_attn_bwd
 * workspace bytes, dK/dV head-split flag, pb_attn_fwd workspace bytes,
 * forward KV chunk (KV tiles per workgroup; 0 = whole lists).  Plans passed
 * to pb_attn_fwd / pb_attn_bwd must be built with these tile sizes.         */
int pb_attn_config(int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t d, int64_t *out);

/* Tile plan of a packed batch (no counterpart table in the reference; it is
 * the kernels' form of BlockMask.{kv,full_kv}_indices (by_kv = 0) or
 * {q,full_q}_indices (by_kv = 1) at the kernel tile sizes):
 *   counts[b][r]            number of non-empty tiles for row tile r
 *   lists[b][r][0..counts)  ascending tile indices, each (tile << 1) | FULL
 * Row tiles are query tiles of q_tile tokens (by_kv = 0) or key tiles of
 * kv_tile tokens (by_kv = 1).  class_ws holds b*nq*nkv bytes.               */
int pb_attn_plan(const int64_t *doc_ids, int64_t doc_stride, int64_t b, int64_t s,
                 int64_t q_tile, int64_t kv_tile, int by_kv, int32_t *counts,
                 int32_t *lists, uint8_t *class_ws, void *stream);

/* Replaces the FlexAttention forward launched at packbalance/model/attention.py:116-122
 * (flex_attention(q, k, v, block_mask=doc mask, enable_gqa=Hq != Hkv)):
 *   out[b,h,i] = sum_j softmax_j(scale * q[b,h,i].k[b,h/G,j] | mask) v[b,h/G,j]
 * with mask(i, j) = doc[b,i] == doc[b,j] && i >= j, G = hq / hkv.
 * q/k/v/out are bf16 (dtype must be PB_BF16), head_dim d <= 128, scale > 0.
 * lse (fp32 [b, hq, s]) receives log2(sum_j exp2(scale*log2(e)*q.k)) for the
 * backward.  plan = pb_attn_plan(by_kv = 0) with the forward tiles of
 * pb_attn_config; workspace: out[8] bytes of pb_attn_config (may be NULL when
 * that is 0).                                                               */
int pb_attn_fwd(const pb_bhsd *q, const pb_bhsd *k, const pb_bhsd *v, const pb_bhsd *out,
                float *lse, void *workspace, const int64_t *doc_ids, int64_t doc_stride,
                const int32_t *plan_counts, const int32_t *plan_lists, int64_t b,
                int64_t hq, int64_t hkv, int64_t s, int64_t d, float scale, int dtype,
                void *stream);

/* Replaces the FlexAttention backward (dQ, dK, dV; dK/dV summed over each
 * GQA group, as enable_gqa does).  workspace: out[6] bytes of pb_attn_config
 * (at head dim 128 on large grids it also holds the bf16 dS blocks of the
 * causal 64 x 64 tiles that dQ is formed from: B * Hkv * T * G * 8 KiB for
 * T = (S/64)(S/64+1)/2, 17.3 GB at B 8, S 8192, Hq 32, Hkv 8; shapes past
 * 32 GiB recompute S and dP for dQ instead).
 * kv_plan = pb_attn_plan(by_kv = 1) with the dK/dV tiles,
 * q_plan  = pb_attn_plan(by_kv = 0) with the dQ tiles of pb_attn_config.     */
int pb_attn_bwd(const pb_bhsd *q, const pb_bhsd *k, const pb_bhsd *v, const pb_bhsd *out,
                const pb_bhsd *dout, const pb_bhsd *dq, const pb_bhsd *dk,
                const pb_bhsd *dv, const float *lse, void *workspace,
                const int64_t *doc_ids, int64_t doc_stride, const int32_t *q_plan_counts,
                const int32_t *q_plan_lists, const int32_t *kv_plan_counts,
                const int32_t *kv_plan_lists, int64_t b, int64_t hq, int64_t hkv, int64_t s,
                int64_t d, float scale, int dtype, void *stream);

/* fp32 attention: replaces FlexAttention on fp32 q/k/v (the reference's
 * non-autocast path, packbalance/model/attention.py:116-122, which computes
 * in fp32 where pb_attn_fwd takes bf16 operands).  Same mask, GQA mapping,
 * scale and log2-domain lse as pb_attn_fwd; q/k/v/out are fp32 pb_bhsd views
 * with unit head-dim stride, head_dim d <= 128; no plans or workspace.  fp32
 * operands on the fp32 matrix cores.                                        */
int pb_attn_fwd_f32(const pb_bhsd *q, const pb_bhsd *k, const pb_bhsd *v, const pb_bhsd *out,
                    float *lse, const int64_t *doc_ids, int64_t doc_stride, int64_t b,
                    int64_t hq, int64_t hkv, int64_t s, int64_t d, float scale, void *stream);

/* Backward of pb_attn_fwd_f32 (FlexAttention's backward on fp32 tensors):
 * dQ, and dK / dV summed over each GQA group, all fp32.  `workspace`:
 * pb_attn_bwd_f32_workspace_bytes bytes, 256-byte aligned: delta =
 * rowsum(dO * O), then on small grids the fp32 dK / dV partials of the KV
 * tiles' chunked walks over heads and query sub-tiles, added in a fixed
 * order (run-to-run deterministic).                                         */
int64_t pb_attn_bwd_f32_workspace_bytes(int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t d);
int pb_attn_bwd_f32(const pb_bhsd *q, const pb_bhsd *k, const pb_bhsd *v, const pb_bhsd *out,
                    const pb_bhsd *dout, const pb_bhsd *dq, const pb_bhsd *dk,
                    const pb_bhsd *dv, const float *lse, void *workspace,
                    const int64_t *doc_ids, int64_t doc_stride, int64_t b, int64_t hq,
                    int64_t hkv, int64_t s, int64_t d, float scale, void *stream);

/* ---- Fused LM-head cross-entropy ----------------------------------------
 * Replaces packbalance/kernels/fused_ce.py:143-217 (_FusedLinearCE /
 * linear_cross_entropy).  x [n, d] and w [v, d] are bf16 with 16-byte aligned
 * rows, d % 8 == 0 (row strides ldx, ldw).  The logits x w^T are computed by
 * bf16 MFMA tiles with fp32 accumulation and reduced in registers; they are
 * never written.  Per row: lse (fp32, natural log) and
 *   loss_rows[r] = lse - logit_t + z*lse^2   (0 if t == ignore_index,
 *                                              NaN if t is outside [0, v)),
 * loss_sum[0] = fixed-order fp32 sum of loss_rows.
 * workspace: pb_lmhead_ce_workspace_bytes(n, v) bytes.                     */
int64_t pb_lmhead_ce_workspace_bytes(int64_t n, int64_t v);
int pb_lmhead_ce_fwd(const void *x, int64_t ldx, const void *w, int64_t ldw, int64_t n,
                     int64_t v, int64_t d, const int64_t *targets, int64_t ignore_index,
                     float z_loss_coeff, float *loss_rows, float *lse, float *loss_sum,
                     void *workspace, void *stream);
/* pb_lmhead_ce_fwd with the logits' precision and storage chosen: with
 * logits_dtype PB_BF16 every logit is rounded to bf16 before lse, the target
 * logit and the loss use it (the reference's `x @ W.T` of bf16 operands, or
 * under bf16 autocast, is a bf16 tensor: fused_ce.py:159, 182); PB_F32 keeps
 * the fp32 accumulators (pb_lmhead_ce_fwd).  With logits != NULL the logits
 * are also written, in logits_dtype, as logits^T [v, ldlg] (vocab-major: row
 * = vocab id; ldlg >= n, ldlg % 8 == 0, 16-byte aligned) for
 * pb_lmhead_ce_bwd_logits.                                                 */
int pb_lmhead_ce_fwd_logits(const void *x, int64_t ldx, const void *w, int64_t ldw, int64_t n,
                            int64_t v, int64_t d, const int64_t *targets, int64_t ignore_index,
                            float z_loss_coeff, float *loss_rows, float *lse, float *loss_sum,
                            void *workspace, int logits_dtype, void *logits, int64_t ldlg,
                            void *stream);

/* Backward of pb_lmhead_ce_fwd (fused_ce.py:176-202), vocab chunk by vocab
 * chunk (vchunk rows of w, a multiple of 8):
 *   dL = (softmax*(1 + 2z*lse) - onehot) * grad_out   (bf16, one chunk)
 *   dx = sum over chunks dL w_chunk   (fp32 accumulation; dx in dx_dtype)
 *   dw[chunk] = dL^T x                (written in dw_dtype; with
 *                                      dw_accumulate != 0, dw must be fp32
 *                                      and the product is added to it)
 * xt = x^T [d, >= n] and wt = w^T [d, >= v] (bf16, e.g. from pb_pack_bf16);
 * workspace: pb_lmhead_ce_bwd_workspace_bytes(n, v, d, vchunk) bytes (the
 * dlogits chunk in both layouts and fp32 dx accumulators).
 * grad_out is a device pointer to one fp32 (no host synchronisation).       */
int64_t pb_lmhead_ce_bwd_workspace_bytes(int64_t n, int64_t v, int64_t d, int64_t vchunk);
int pb_lmhead_ce_bwd(const void *x, int64_t ldx, const void *w, int64_t ldw, const void *xt,
                     int64_t ldxt, const void *wt, int64_t ldwt, int64_t n, int64_t v,
                     int64_t d, const int64_t *targets, int64_t ignore_index,
                     float z_loss_coeff, const float *lse, const float *grad_out,
                     int64_t vchunk, void *workspace, void *dx, int dx_dtype, int64_t lddx,
                     void *dw, int dw_dtype, int64_t lddw, int dw_accumulate,
                     void *stream);
/* Backward of pb_lmhead_ce_fwd_logits (same x, w, targets, lse, and the
 * forward's logits_dtype).  logits == NULL: the logits are recomputed (and
 * rounded to bf16 for PB_BF16) as in pb_lmhead_ce_bwd.  Otherwise each
 * chunk's dlogits come from one memory-bound pass over the stored logits^T
 * instead of the recomputing GEMM (2 n v d FLOPs fewer); the dx and dW
 * products are those of pb_lmhead_ce_bwd.  Stored logits need
 * (n + 127) / 128 <= 65535.                                                */
int pb_lmhead_ce_bwd_logits(const void *x, int64_t ldx, const void *w, int64_t ldw,
                            const void *xt, int64_t ldxt, const void *wt, int64_t ldwt,
                            int64_t n, int64_t v, int64_t d, const int64_t *targets,
                            int64_t ignore_index, float z_loss_coeff, const float *lse,
                            const float *grad_out, int64_t vchunk, void *workspace, void *dx,
                            int dx_dtype, int64_t lddx, void *dw, int dw_dtype, int64_t lddw,
                            int dw_accumulate, int logits_dtype, const void *logits,
                            int64_t ldlg, void *stream);

/* One vocab chunk of the backward's dlogits (no reference counterpart: the
 * dL step of pb_lmhead_ce_bwd / _logits, fused_ce.py:176-202, for callers
 * that run the dx and dW products on a GEMM library -- the Python layer runs
 * them through torch on hipBLASLt):
 *   dL [n][vc] (row stride ldl) and dL^T [vc][n] (row stride ldlt), bf16,
 *   of vocab rows v0 .. v0 + vc - 1 (v0 + vc <= v),
 * from the stored logits^T of pb_lmhead_ce_fwd_logits (logits != NULL, its
 * logits_dtype) or by recomputing them (rounded to bf16 for PB_BF16), with
 * the lse of the forward and grad_out a device pointer to one fp32.  x, w,
 * dl and dlt 16-byte aligned with row strides % 8 == 0, d % 8 == 0.        */
int pb_lmhead_ce_dlogits(const void *x, int64_t ldx, const void *w, int64_t ldw, int64_t n,
                         int64_t v, int64_t d, const int64_t *targets, int64_t ignore_index,
                         float z_loss_coeff, const float *lse, const float *grad_out,
                         int64_t v0, int64_t vc, void *dl, int64_t ldl, void *dlt, int64_t ldlt,
                         int logits_dtype, const void *logits, int64_t ldlg, void *stream);

/* ---- Fused residual add + RMSNorm (per-operand dtypes) ------------------
 * Replaces the decoder's `hidden = hidden + sublayer_out` followed by the
 * next rmsnorm (packbalance/model/llama.py:122-125 with
 * packbalance/kernels/rmsnorm.py:77-125), and the autocast casts around it:
 *   h = x + delta  (delta may be NULL: h = x),  written to h_out in x_dtype
 *   (h_out may be NULL or alias x);  y = h * rstd * w in y_dtype;
 *   rstd[rows] fp32.
 * Backward (workspace: pb_add_rmsnorm_bwd_workspace_bytes):
 *   d = rstd*(dy*w - h_hat*mean(dy*w*h_hat)) + dres  (dres may be NULL)
 *   dx = d in h_dtype, ddelta = d in ddelta_dtype (may be NULL),
 *   dw = sum_rows dy*h_hat in w_dtype (dw_accumulate != 0: fp32 w and dw,
 *   and the sum is added to dw).   dx may alias dres.
 * Unit inner stride; row strides in elements.                                */
int pb_add_rmsnorm_fwd(const void *x, int64_t x_row_stride, int x_dtype, const void *delta,
                       int64_t delta_row_stride, int delta_dtype, void *h_out,
                       int64_t h_row_stride, const void *w, int w_dtype, void *y,
                       int64_t y_row_stride, int y_dtype, float *rstd, int64_t rows, int64_t n,
                       float eps, void *stream);
int64_t pb_add_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t n);
int pb_add_rmsnorm_bwd(const void *dy, int64_t dy_row_stride, int dy_dtype, const void *h,
                       int64_t h_row_stride, int h_dtype, const void *w, int w_dtype,
                       const float *rstd, const void *dres, int64_t dres_row_stride, void *dx,
                       int64_t dx_row_stride, void *ddelta, int64_t ddelta_row_stride,
                       int ddelta_dtype, void *dw, int dw_accumulate, void *workspace,
                       int64_t rows, int64_t n, void *stream);

/* The same backward with the dw reduction left to the caller (no reference
 * counterpart: the reference's rmsnorm backward sums dw in a second PyTorch
 * pass, packbalance/kernels/rmsnorm.py:106-118, once per norm).  dx and
 * ddelta as pb_add_rmsnorm_bwd; `partials` (pb_add_rmsnorm_bwd_workspace_bytes
 * bytes) receives the fp32 per-workgroup partial rows of dw.
 * pb_rmsnorm_dw_reduce_batched then adds, for i < count, the column sums of
 * the table at partials + i * problem_stride (floats) to the fp32 dw[i]
 * (a host array of count device pointers), each problem's table written by
 * pb_add_rmsnorm_bwd_partials with the same rows and n -- one launch per 32
 * problems instead of one per norm, with the same bits as dw_accumulate.   */
int pb_add_rmsnorm_bwd_partials(const void *dy, int64_t dy_row_stride, int dy_dtype,
                                const void *h, int64_t h_row_stride, int h_dtype, const void *w,
                                int w_dtype, const float *rstd, const void *dres,
                                int64_t dres_row_stride, void *dx, int64_t dx_row_stride,
                                void *ddelta, int64_t ddelta_row_stride, int ddelta_dtype,
                                float *partials, int64_t rows, int64_t n, void *stream);
int pb_rmsnorm_dw_reduce_batched(const float *partials, int64_t problem_stride,
                                 float *const *dw, int64_t count, int64_t rows, int64_t n,
                                 void *stream);

/* ---- Model inputs of packs, built on the device --------------------------
 * Replaces packbalance/data/dataset.py:33-76 (PackedDataset.__getitem__) for
 * a batch of packs, reading a token store resident in device memory (the
 * tokens.bin of data/store.py:12-56; store_elem_bytes 2 = uint16, 4 =
 * uint32, 8 = int64).  Pack p's segments are (seg_start[i], seg_len[i]) for
 * i in [pack_seg[p], pack_seg[p+1]) (at most max_segs <= 4096 per pack).
 * Outputs int64 [n_packs, total], total = seq_len (rows == 0: packed, the
 * segments back to back from position 0) or rows * seq_len (rows > 0:
 * padded, segment i in row i and the whole row one document):
 *   input_ids = tokens, labels = next token of the same segment (-100 on its
 *   last token), position_ids = 0..len-1, doc_ids = segment index;
 *   pad_token_id / -100 / 0 / -1 at every other position.
 * The caller validates the table (segments inside the store, packs within
 * total); the kernel keeps every access in bounds regardless.              */
int pb_pack_tensors(const void *store, int store_elem_bytes, int64_t store_len,
                    const int64_t *seg_start, const int64_t *seg_len, const int64_t *pack_seg,
                    int64_t n_packs, int64_t max_segs, int64_t seq_len, int64_t rows,
                    int64_t pad_token_id, int64_t *input_ids, int64_t *labels,
                    int64_t *position_ids, int64_t *doc_ids, void *stream);

/* ---- Clip-by-global-norm + AdamW over one flat fp32 buffer --------------
 * Replaces torch.nn.utils.clip_grad_norm_(params, max_grad_norm) followed by
 * torch.optim.AdamW(params, lr, (beta1, beta2), eps, weight_decay,
 * fused=True).step() as the reference's train loop calls them
 * (packbalance/train/train.py:58-69,353-362; profiling/bench_train.py:79-85,
 * 115-116), for uniform hyper-parameters over parameters stored as one flat
 * buffer:
 *   grad = sum of grad_slots buffers grad_slot_stride elements apart (one
 *   per concurrently run micro-batch, say); with more than one slot the sum
 *   is written back into slot 0 (grad[0..n));
 *   norm = ||grad||_2 -> *grad_norm_out (may be NULL);
 *   c = min(max_grad_norm / (norm + 1e-6), 1)  (1 when max_grad_norm <= 0);
 *   *step += 1 (device fp32, the optimizer's step count);
 *   p -= lr*wd*p;  m = b1 m + (1-b1) c g;  v = b2 v + (1-b2) (c g)^2;
 *   p -= lr/(1-b1^t) * m / (sqrt(v)/sqrt(1-b2^t) + eps);
 *   param_copy (may be NULL) = p rounded to copy_dtype.
 * The clipped gradient is not stored back.
 * Buffers 16-byte aligned (param_copy 8-byte); workspace:
 * pb_clip_adamw_workspace_bytes(n) bytes, 16-byte aligned.                  */
int64_t pb_clip_adamw_workspace_bytes(int64_t n);
int pb_clip_adamw_step(float *param, float *grad, int grad_slots, int64_t grad_slot_stride,
                       float *exp_avg, float *exp_avg_sq, void *param_copy, int copy_dtype,
                       int64_t n, float lr, float beta1, float beta2, float eps,
                       float weight_decay, float max_grad_norm, float *step,
                       float *grad_norm_out, void *workspace, void *stream);

/* ---- Rotary position embedding (q and k in one launch) ------------------
 * Replaces packbalance/model/rope.py:34-42 (apply_rotary_pos_emb, NeoX
 * rotate_half).  q [b, hq, s, d] and k [b, hkv, s, d] are pb_bhsd views with
 * a contiguous head dim (d even); q_out / k_out may alias q / k.  cos and
 * sin are fp32 [b, s, d/2] (already gathered by position id, rope.py:26) with
 * a contiguous last dim and the given b / s strides.  inverse = 0 rotates by
 * +theta (forward), inverse = 1 by -theta (the backward of the forward).
 * Arithmetic is fp32 with one rounding to dtype.                            */
int pb_rope_qk(const pb_bhsd *q, const pb_bhsd *k, const pb_bhsd *q_out, const pb_bhsd *k_out,
               const float *cos, int64_t cos_stride_b, int64_t cos_stride_s, const float *sin,
               int64_t sin_stride_b, int64_t sin_stride_s, int64_t b, int64_t s, int64_t hq,
               int64_t hkv, int64_t d, int dtype, int inverse, void *stream);

/* Layout helper of the CE path: dst (bf16) <- src (any float dtype), cast
 * and, if transpose, transposed; dst is [dst_rows, dst_cols] with row stride
 * dst_ld, and every dst element outside the copied [rows, cols] (or
 * [cols, rows]) block is written as zero (padding).  No reference
 * counterpart: it feeds the K-contiguous operands the MFMA tiles read.      */
int pb_pack_bf16(const void *src, int src_dtype, int64_t src_ld, int64_t rows, int64_t cols,
                 void *dst, int64_t dst_ld, int64_t dst_rows, int64_t dst_cols, int transpose,
                 void *stream);

/* Batched transpose: dst[b][c][r] = src[b][r][c] for b < batch, r < rows,
 * c < cols; src rows src_row_stride and matrices src_batch_stride elements
 * apart, dst contiguous [batch, cols, rows]; 2- or 4-byte elements (bits
 * copied).  No reference counterpart: it writes the transposed weight copies
 * that the input-gradient GEMMs read (the reference's nn.Linear backward
 * reads W as stored).                                                       */
int pb_transpose_batched(const void *src, int64_t src_batch_stride, int64_t src_row_stride,
                         void *dst, int64_t batch, int64_t rows, int64_t cols, int elem_bytes,
                         void *stream);

#ifdef __cplusplus
}
#endif

#endif /* PACKBALANCE_AMD_H */
