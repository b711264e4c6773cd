"""Fused linear cross-entropy on gfx950.

``linear_cross_entropy(x, weight, targets, *, chunk_size=1024,
ignore_index=-100, z_loss_coeff=0.0)`` has the contract of the reference
``packbalance/kernels/fused_ce.py:205-217``: the SUM over rows with target !=
ignore_index of ``lse(x W^T) - (x W^T)_t + z*lse^2``; backward returns ``dx`` in
x's dtype and original shape and ``dw`` in W's dtype (fp32 accumulation).

Forward: one MFMA GEMM kernel computes logits tiles in registers and keeps
only per-token (max, sum-exp) partials and the target logit, then a combine
kernel gives lse and the loss.  The logits have the precision of the
reference's ``x @ W.T`` (``logits_dtype_for``): bf16 for two bf16 operands or
under bf16 autocast (each logit rounded to bf16 before lse, loss and
dlogits), fp32 otherwise.  By default nothing else is kept: as in the
reference, the full logits are never materialised and the backward recomputes
them.  A caller with memory to spare may raise the logits budget
(``logits_budget`` / ``LOGITS_BUDGET``, in bytes; cfg4's 16384 x 128256 bf16
logits are 4.2 GB of the 288 GB of HBM): a forward whose logits fit then also
writes them (vocab-major) and keeps them for the backward, which skips the
recomputing GEMM (same numerics either way).  Backward
streams the vocabulary in chunks (``vocab_chunk``: as many vocab rows as keep
one dlogits chunk of all tokens under ``CHUNK_BUDGET`` elements -- 1 GiB of
bf16 per layout -- but at least 8192): the chunk's dlogits (bf16) come from
one memory-bound pass over the stored logits, or from a GEMM that recomputes
them (the kernel of ``pb_lmhead_ce_dlogits``), then two plain library GEMMs
(torch on hipBLASLt) accumulate dx and write the chunk's dW rows; the C
boundary's ``pb_lmhead_ce_bwd`` runs the same steps with this build's own
GEMMs for C callers, and so does ``linear_cross_entropy_accumulate`` (the
training step's form, run on two streams at once inside a captured graph).  Fewer, longer chunks mean fewer passes over the fp32 dx
accumulator (cfg4: 4 chunks of 32768 rows instead of 16 of 8192).
Operands are bf16 with fp32 accumulation (as the reference's autocast GEMM
rounds them), except for fp32 x and W outside bf16 autocast: there the
reference's logits are an fp32 product, and so are these (``_LinearCEF32``:
fp32 library GEMMs over token-row chunks with the row CE kernel).  ``chunk_size`` (token rows per
chunk in the reference) is accepted and validated; memory is bounded by the
vocab chunk instead.

``ce_rows`` is the contract of the reference's ``_ce_launch`` / ``_ce_kernel``
(``fused_ce.py:31-118``): per-row loss (and optionally dlogits) over a
materialised ``[M, V]`` logits block with any strides.
"""

from __future__ import annotations

import torch

from packbalance_amd import _native as N

HAS_NATIVE = N.available()
HAS_TRITON = HAS_NATIVE


def use_triton(x: torch.Tensor) -> bool:
    """Reference name (fused_ce.py:139-140): True when the native kernels serve ``x``."""
    return HAS_NATIVE and x.is_cuda


def ce_rows(logits: torch.Tensor, targets: torch.Tensor, *, write_dlogits: bool,
            ignore_index: int = -100, z_loss_coeff: float = 0.0,
            dlogits_dtype: torch.dtype | None = None):
    """Per-row CE of a logits block: returns (loss fp32 [M], lse fp32 [M], dlogits | None).

    dlogits has the dtype and strides of ``logits`` (``torch.empty_like``), or
    is a contiguous tensor of ``dlogits_dtype`` when that is given.
    """
    N.require_device(logits, targets, op="ce_rows")
    if logits.dim() != 2:
        raise ValueError("ce_rows expects [M, V] logits")
    m, v = logits.shape
    t = targets.reshape(-1)
    if t.numel() != m:
        raise ValueError(f"logits has {m} rows but targets has {t.numel()}")
    t = t.to(torch.int64).contiguous()
    dl = None
    if write_dlogits and dlogits_dtype is not None:
        dl = torch.empty((m, v), dtype=dlogits_dtype, device=logits.device)
    elif write_dlogits:
        dl = torch.empty_like(logits)
        if dl.stride() != logits.stride():  # non-dense view: the kernel shares strides
            logits = logits.contiguous()
            dl = torch.empty_like(logits)
    loss = torch.empty(m, dtype=torch.float32, device=logits.device)
    lse = torch.empty(m, dtype=torch.float32, device=logits.device)
    dls = dl.stride() if dl is not None else logits.stride()
    N.call(
        "pb_ce_rows_dl",
        logits.data_ptr(), logits.stride(0), logits.stride(1), N.dtype_code(logits),
        t.data_ptr(), loss.data_ptr(), lse.data_ptr(), N.ptr(dl), dls[0], dls[1],
        N.dtype_code(dl if dl is not None else logits), m, v, int(ignore_index),
        float(z_loss_coeff), N.stream_ptr(logits),
    )
    return loss, lse, dl


VOCAB_CHUNK = 8192
CHUNK_BUDGET = 1 << 29  # dlogits elements per chunk (1 GiB of bf16 per layout)
_chunk_rows: int | None = None  # set by vocab_chunk_rows()


def _round8(n: int) -> int:
    return (n + 7) // 8 * 8


LOGITS_BUDGET = 0  # bytes of logits a forward may keep for its backward (0: never)
_logits_budget: int | None = None  # set by logits_budget()


def logits_dtype_for(x_dtype: torch.dtype, w_dtype: torch.dtype) -> torch.dtype:
    """Precision of the logits: that of the reference's ``x @ W.T`` (fused_ce.py:159, 182),
    bf16 for two bf16 operands or under bf16 autocast, else fp32 (fp16 operands, which the
    kernels round to bf16 like every operand, keep fp32 logits)."""
    if x_dtype == torch.bfloat16 and w_dtype == torch.bfloat16:
        return torch.bfloat16
    if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16:
        return torch.bfloat16
    return torch.float32


def stores_logits(n: int, v: int, dtype: torch.dtype = torch.bfloat16) -> bool:
    """True when a forward over n tokens and v vocab rows keeps its logits (of ``dtype``)."""
    budget = LOGITS_BUDGET if _logits_budget is None else _logits_budget
    return n > 0 and v * _round8(n) * torch.tensor([], dtype=dtype).element_size() <= budget


class logits_budget:
    """Context manager: forwards started inside it keep their logits only when they fit
    ``nbytes`` (0: never, so the backward recomputes them); ``None`` restores
    ``LOGITS_BUDGET``."""

    def __init__(self, nbytes: int | None) -> None:
        if nbytes is not None and int(nbytes) < 0:
            raise ValueError("logits budget must be >= 0 bytes")
        self.nbytes = None if nbytes is None else int(nbytes)

    def __enter__(self):
        global _logits_budget
        self._saved, _logits_budget = _logits_budget, self.nbytes
        return self

    def __exit__(self, *exc) -> None:
        global _logits_budget
        _logits_budget = self._saved


def _lg_code(dtype: torch.dtype) -> int:
    return N.PB_BF16 if dtype == torch.bfloat16 else N.PB_F32


def _ce_forward(xb, wb, t, n, v, d8, ignore_index, z, rows, lse, total, dev, stream, lg_dtype):
    """Forward launch; returns the stored logits^T [v, round8(n)] (of lg_dtype) or None."""
    ws = torch.empty(max(1, N.lib().pb_lmhead_ce_workspace_bytes(n, v) // 4),
                     dtype=torch.float32, device=dev)
    lg = None
    if stores_logits(n, v, lg_dtype):
        lg = torch.empty((v, _round8(n)), dtype=lg_dtype, device=dev)
    N.call("pb_lmhead_ce_fwd_logits", xb.data_ptr(), xb.stride(0), wb.data_ptr(), wb.stride(0),
           n, v, d8, t.data_ptr(), ignore_index, z, rows.data_ptr(), lse.data_ptr(),
           total.data_ptr(), ws.data_ptr(), _lg_code(lg_dtype), N.ptr(lg),
           lg.stride(0) if lg is not None else 0, stream)
    return lg


def _ce_backward_kernels(xb, wb, xt, wt, t, lse, go, lg, lg_dtype, n, v, d8, ignore_index, z,
                         vchunk, dx, dw, dw_accumulate):
    """Backward on this build's own kernels (``pb_lmhead_ce_bwd_logits``: dlogits and the
    dx / dW DMA GEMMs, which read the transposed ``xt`` and ``wt``): the training step's
    path, whose two micro-batch streams run it concurrently inside one captured graph."""
    ws = torch.empty(N.lib().pb_lmhead_ce_bwd_workspace_bytes(n, v, d8, vchunk),
                     dtype=torch.uint8, device=xb.device)
    N.call("pb_lmhead_ce_bwd_logits", xb.data_ptr(), xb.stride(0), wb.data_ptr(), wb.stride(0),
           xt.data_ptr(), xt.stride(0), wt.data_ptr(), wt.stride(0), n, v, d8, t.data_ptr(),
           ignore_index, z, lse.data_ptr(), go.data_ptr(), vchunk, ws.data_ptr(), dx.data_ptr(),
           N.dtype_code(dx), dx.stride(0), dw.data_ptr(),
           N.PB_F32 if dw_accumulate else N.dtype_code(dw), dw.stride(0), int(dw_accumulate),
           _lg_code(lg_dtype), N.ptr(lg), lg.stride(0) if lg is not None else 0,
           N.stream_ptr(xb))


def _ce_backward(xb, wb, t, lse, go, lg, lg_dtype, n, v, d8, ignore_index, z, vchunk, dx, dw,
                 dw_accumulate):
    """Backward, vocab chunk by vocab chunk: the chunk's dL [n, vc] and dL^T [vc, n]
    (bf16) from ``pb_lmhead_ce_dlogits`` -- from the stored logits ``lg`` when given,
    else recomputing them --, then dx (+)= dL W_chunk into an fp32 accumulator and
    dW_chunk (+)= dL^T x as library GEMMs (torch -> hipBLASLt, fp32 accumulation),
    which run these plain products faster than this build's own DMA GEMM
    (``pb_lmhead_ce_bwd``; at a cfg4 chunk dx 977 vs 1,110 us and dW 809 vs 967 us)
    and read x and W as they are, with no transposed copies."""
    dev = xb.device
    stream = N.stream_ptr(xb)
    dl = torch.empty((n, vchunk), dtype=torch.bfloat16, device=dev)
    dlt = torch.empty((vchunk, _round8(n)), dtype=torch.bfloat16, device=dev)
    acc = dx if dx.dtype == torch.float32 else torch.empty((n, d8), dtype=torch.float32,
                                                           device=dev)
    for c, v0 in enumerate(range(0, v, vchunk)):
        vc = min(vchunk, v - v0)
        N.call("pb_lmhead_ce_dlogits", xb.data_ptr(), xb.stride(0), wb.data_ptr(), wb.stride(0),
               n, v, d8, t.data_ptr(), ignore_index, z, lse.data_ptr(), go.data_ptr(), v0, vc,
               dl.data_ptr(), dl.stride(0), dlt.data_ptr(), dlt.stride(0), _lg_code(lg_dtype),
               N.ptr(lg), lg.stride(0) if lg is not None else 0, stream)
        dlc, dltc, dwc = dl[:, :vc], dlt[:vc, :n], dw[v0:v0 + vc]
        # beta 0 on the first chunk: the accumulator's old contents are not read
        torch.addmm(acc, dlc, wb[v0:v0 + vc], beta=0 if c == 0 else 1,
                    out_dtype=torch.float32, out=acc)
        if dw_accumulate or dwc.dtype == torch.float32:
            torch.addmm(dwc, dltc, xb, beta=1 if dw_accumulate else 0, out_dtype=torch.float32,
                        out=dwc)
        elif dwc.dtype == torch.bfloat16:
            torch.mm(dltc, xb, out=dwc)
        else:  # fp16 weights: the product in fp32, rounded once
            dwc.copy_(torch.addmm(torch.empty((vc, d8), dtype=torch.float32, device=dev), dltc, xb,
                                  beta=0, out_dtype=torch.float32))
    if acc is not dx:
        dx.copy_(acc)


def vocab_chunk(n: int, v: int) -> int:
    """Vocab rows per backward chunk: >= VOCAB_CHUNK, all of v if n*v fits the budget
    (or the fixed count set by ``vocab_chunk_rows``, capped at v)."""
    if _chunk_rows is not None:
        return min(_round8(v), _chunk_rows)
    fit = (CHUNK_BUDGET // max(1, n)) // 8 * 8
    return min(_round8(v), max(VOCAB_CHUNK, fit))


class vocab_chunk_rows:
    """Context manager: backward passes started inside it stream the vocabulary in
    chunks of exactly ``rows`` vocab rows (a multiple of 8), e.g. a benchmark's
    stated chunk size.  The public signature of ``linear_cross_entropy`` is
    unchanged; ``None`` restores the default budget rule."""

    def __init__(self, rows: int | None) -> None:
        if rows is not None and (int(rows) <= 0 or int(rows) % 8):
            raise ValueError("vocab chunk rows must be a positive multiple of 8")
        self.rows = None if rows is None else int(rows)

    def __enter__(self):
        global _chunk_rows
        self._saved, _chunk_rows = _chunk_rows, self.rows
        return self

    def __exit__(self, *exc) -> None:
        global _chunk_rows
        _chunk_rows = self._saved


def _bf16_rows(t: torch.Tensor) -> torch.Tensor:
    """t [rows, k] as bf16 rows with 16-byte aligned starts and k padded to a multiple of 8."""
    rows, k = t.shape
    if (t.dtype == torch.bfloat16 and t.stride(1) == 1 and k % 8 == 0 and t.stride(0) % 8 == 0
            and t.data_ptr() % 16 == 0):
        return t
    k8 = _round8(k)
    out = torch.empty((rows, k8), dtype=torch.bfloat16, device=t.device)
    src = t if t.stride(1) == 1 else t.contiguous()
    N.call("pb_pack_bf16", src.data_ptr(), N.dtype_code(src), src.stride(0), rows, k,
           out.data_ptr(), k8, rows, k8, 0, N.stream_ptr(t))
    return out


def _transpose_bf16(t: torch.Tensor) -> torch.Tensor:
    """t [rows, k] bf16 -> [k, round8(rows)] bf16, zero-padded."""
    rows, k = t.shape
    r8 = _round8(rows)
    out = torch.empty((k, r8), dtype=torch.bfloat16, device=t.device)
    N.call("pb_pack_bf16", t.data_ptr(), N.PB_BF16, t.stride(0), rows, k, out.data_ptr(), r8,
           k, r8, 1, N.stream_ptr(t))
    return out


class _FusedLinearCE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, targets, chunk_size, ignore_index, z_loss_coeff):
        x2d = x.reshape(-1, x.shape[-1])
        t1d = targets.reshape(-1)
        if x2d.shape[0] != t1d.shape[0]:
            raise ValueError(f"x has {x2d.shape[0]} rows but targets has {t1d.shape[0]}")
        if weight.dim() != 2 or weight.shape[1] != x2d.shape[1]:
            raise ValueError(f"weight {tuple(weight.shape)} does not match x features {x2d.shape[1]}")
        n, d = x2d.shape
        v = weight.shape[0]
        dev = x.device
        t = t1d.to(torch.int64).contiguous()
        total = torch.zeros((), dtype=torch.float32, device=dev)
        ctx.x_shape, ctx.x_dtype, ctx.w_dtype, ctx.d = x.shape, x.dtype, weight.dtype, d
        ctx.ignore_index, ctx.z = int(ignore_index), float(z_loss_coeff)
        if n == 0:
            ctx.save_for_backward(x2d, weight, t, total, None)
            ctx.empty = True
            return total
        ctx.empty = False
        xb = _bf16_rows(x2d)
        wb = _bf16_rows(weight)
        lse = torch.empty(n, dtype=torch.float32, device=dev)
        rows = torch.empty(n, dtype=torch.float32, device=dev)
        ctx.lg_dtype = logits_dtype_for(x.dtype, weight.dtype)
        lg = _ce_forward(xb, wb, t, n, v, xb.shape[1], ctx.ignore_index, ctx.z, rows, lse,
                         total, dev, N.stream_ptr(x), ctx.lg_dtype)
        ctx.save_for_backward(xb, wb, t, lse, lg)
        return total

    @staticmethod
    def backward(ctx, grad_output):
        xb, wb, t, lse, lg = ctx.saved_tensors
        if ctx.empty:
            dw = torch.zeros(wb.shape, dtype=ctx.w_dtype, device=wb.device)
            return (torch.zeros(ctx.x_shape, dtype=ctx.x_dtype, device=xb.device), dw,
                    None, None, None, None)
        n, d8 = xb.shape
        v = wb.shape[0]
        dev = xb.device
        vchunk = vocab_chunk(n, v)
        dx = torch.empty((n, d8), dtype=ctx.x_dtype, device=dev)
        dw = torch.empty((v, d8), dtype=ctx.w_dtype, device=dev)
        go = grad_output.detach().to(torch.float32).reshape(1).contiguous()
        _ce_backward(xb, wb, t, lse, go, lg, ctx.lg_dtype, n, v, d8, ctx.ignore_index, ctx.z,
                     vchunk, dx, dw, False)
        d = ctx.d
        if d8 != d:
            dx, dw = dx[:, :d], dw[:, :d]
        return dx.reshape(ctx.x_shape), dw, None, None, None, None


F32_CHUNK_BYTES = 1 << 30  # fp32 logits per row chunk of the fp32 path


class _LinearCEF32(torch.autograd.Function):
    """fp32 x and W without bf16 autocast: the reference computes ``x @ W.T`` in fp32
    (fused_ce.py:159, 182), so the logits here are fp32 library GEMMs over token-row
    chunks, with the row CE kernel (``ce_rows``) for loss, lse and dlogits."""

    @staticmethod
    def forward(ctx, x, weight, targets, ignore_index, z_loss_coeff):
        x2d = x.reshape(-1, x.shape[-1]).to(torch.float32)
        w = weight.to(torch.float32)
        t = targets.reshape(-1).to(torch.int64).contiguous()
        n, v = x2d.shape[0], w.shape[0]
        rows = max(1, F32_CHUNK_BYTES // (4 * v))
        total = torch.zeros((), dtype=torch.float32, device=x.device)
        for r0 in range(0, n, rows):
            logits = x2d[r0:r0 + rows] @ w.t()
            loss, _, _ = ce_rows(logits, t[r0:r0 + rows], write_dlogits=False,
                                 ignore_index=ignore_index, z_loss_coeff=z_loss_coeff)
            total = total + loss.sum()
        ctx.save_for_backward(x2d, w, t)
        ctx.meta = (x.shape, x.dtype, weight.dtype, rows, int(ignore_index), float(z_loss_coeff))
        return total

    @staticmethod
    def backward(ctx, grad_output):
        x2d, w, t = ctx.saved_tensors
        x_shape, x_dtype, w_dtype, rows, ignore_index, z = ctx.meta
        dx = torch.empty_like(x2d)
        dw = torch.zeros_like(w)
        for r0 in range(0, x2d.shape[0], rows):
            xs = x2d[r0:r0 + rows]
            _, _, dl = ce_rows(xs @ w.t(), t[r0:r0 + rows], write_dlogits=True,
                               ignore_index=ignore_index, z_loss_coeff=z)
            dx[r0:r0 + rows] = dl @ w
            dw.addmm_(dl.t(), xs)
        g = grad_output.to(torch.float32)
        return ((dx * g).to(x_dtype).reshape(x_shape), (dw * g).to(w_dtype), None, None, None)


def _fp32_operands(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """fp32 (or fp64) operands whose logits the reference computes in fp32."""
    wide = (torch.float32, torch.float64)
    return (x.dtype in wide and weight.dtype in wide
            and logits_dtype_for(x.dtype, weight.dtype) == torch.float32)


class _LMHeadCEAccum(torch.autograd.Function):
    """``_FusedLinearCE`` over a caller-held bf16 weight ``wb`` [V, d8] and its transpose
    ``wt`` [d8, >= V], adding dW (fp32) into ``dw_acc`` instead of returning it.  The
    backward runs on this build's own kernels (``_ce_backward_kernels``), not the library
    GEMMs of ``linear_cross_entropy``: the training step runs it on two streams at once
    inside one captured graph, and with the library's long-K products there the step did
    not complete."""

    @staticmethod
    def forward(ctx, x, wb, wt, dw_acc, targets, ignore_index, z_loss_coeff, weight_dtype):
        x2d = x.reshape(-1, x.shape[-1])
        t = targets.reshape(-1).to(torch.int64).contiguous()
        n, d = x2d.shape
        v, d8 = wb.shape
        if t.shape[0] != n or d8 != _round8(d) or dw_acc.shape[0] != v or dw_acc.shape[1] < d:
            raise ValueError("lmhead CE: x / weight / targets / dW shapes disagree")
        if dw_acc.dtype != torch.float32 or dw_acc.stride(1) != 1:
            raise ValueError("lmhead CE: dW accumulator must be fp32 with unit column stride")
        dev = x.device
        total = torch.zeros((), dtype=torch.float32, device=dev)
        xb = _bf16_rows(x2d)
        lse = torch.empty(n, dtype=torch.float32, device=dev)
        rows = torch.empty(n, dtype=torch.float32, device=dev)
        ctx.lg_dtype = logits_dtype_for(x.dtype, weight_dtype)
        lg = _ce_forward(xb, wb, t, n, v, d8, int(ignore_index), float(z_loss_coeff), rows, lse,
                         total, dev, N.stream_ptr(x), ctx.lg_dtype)
        ctx.save_for_backward(xb, wb, wt, t, lse, lg)
        ctx.dw_acc, ctx.x_shape, ctx.x_dtype, ctx.d = dw_acc, x.shape, x.dtype, d
        ctx.ignore_index, ctx.z = int(ignore_index), float(z_loss_coeff)
        return total

    @staticmethod
    def backward(ctx, grad_output):
        xb, wb, wt, t, lse, lg = ctx.saved_tensors
        n, d8 = xb.shape
        v = wb.shape[0]
        dev = xb.device
        dw = ctx.dw_acc
        if dw.shape[1] != d8:
            raise ValueError("lmhead CE: dW accumulator width must equal the padded feature count")
        xt = _transpose_bf16(xb)
        vchunk = vocab_chunk(n, v)
        dx = torch.empty((n, d8), dtype=ctx.x_dtype, device=dev)
        go = grad_output.detach().to(torch.float32).reshape(1).contiguous()
        _ce_backward_kernels(xb, wb, xt, wt, t, lse, go, lg, ctx.lg_dtype, n, v, d8,
                             ctx.ignore_index, ctx.z, vchunk, dx, dw, True)
        if d8 != ctx.d:
            dx = dx[:, :ctx.d]
        return dx.reshape(ctx.x_shape), None, None, None, None, None, None, None


def lmhead_weight_bf16(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(wb, wt): ``weight`` as bf16 rows [V, round8(d)] and their transpose [round8(d), round8(V)],
    to be computed once and passed to ``linear_cross_entropy_accumulate`` while weight is unchanged."""
    wb = _bf16_rows(weight)
    return wb, _transpose_bf16(wb)


def linear_cross_entropy_accumulate(x: torch.Tensor, wb: torch.Tensor, wt: torch.Tensor,
                                    dw_acc: torch.Tensor, targets: torch.Tensor,
                                    *, ignore_index: int = -100,
                                    z_loss_coeff: float = 0.0,
                                    weight_dtype: torch.dtype | None = None) -> torch.Tensor:
    """``linear_cross_entropy`` for a training loop that owns the weight's bf16 copy.

    The forward and loss are those of ``linear_cross_entropy(x, W)`` with ``(wb, wt) =
    lmhead_weight_bf16(W)`` and ``weight_dtype`` = W's dtype (default: wb's, bf16), which
    with x's dtype sets the logits' precision; the backward returns dx and ADDS dW (fp32)
    into ``dw_acc`` [V, d] (d a multiple of 8) instead of returning it.
    """
    N.require_device(x, wb, targets, op="linear_cross_entropy_accumulate")
    return _LMHeadCEAccum.apply(x, wb, wt, dw_acc, targets, ignore_index, z_loss_coeff,
                                wb.dtype if weight_dtype is None else weight_dtype)


def linear_cross_entropy(
    x: torch.Tensor,
    weight: torch.Tensor,
    targets: torch.Tensor,
    *,
    chunk_size: int = 1024,
    ignore_index: int = -100,
    z_loss_coeff: float = 0.0,
) -> torch.Tensor:
    """Return the summed CE loss for ``x @ weight.T`` without full logits (gfx950 kernels;
    a caller may let them be kept for the backward with ``logits_budget``)."""
    N.require_device(x, weight, targets, op="linear_cross_entropy")
    if int(chunk_size) <= 0:
        raise ValueError("chunk_size must be positive")
    if _fp32_operands(x, weight):
        if x.shape[-1] != weight.shape[-1] or weight.dim() != 2:
            raise ValueError(f"weight {tuple(weight.shape)} does not match x features {x.shape[-1]}")
        if x.numel() // max(1, x.shape[-1]) != targets.numel():
            raise ValueError(f"x has {x.numel() // max(1, x.shape[-1])} rows but targets has "
                             f"{targets.numel()}")
        return _LinearCEF32.apply(x, weight, targets, ignore_index, z_loss_coeff)
    return _FusedLinearCE.apply(x, weight, targets, int(chunk_size), ignore_index, z_loss_coeff)
