"""Fused RMSNorm on the gfx950 kernels of ``libpackbalance_amd.so``.

Same public API as the reference ``packbalance/kernels/rmsnorm.py:122-125``
(``rmsnorm(x, weight, eps)``) with the autograd contract of ``_RMSNorm``
(``rmsnorm.py:77-119``): fp32 statistics, ``rstd`` cached for backward, ``y``
and ``dx`` in the activation dtype, ``dw`` accumulated in fp32 and returned in
the weight dtype.  The backward is one fused kernel (``dx`` plus per-block
``dw`` partials) and a small reduction, instead of the reference's Triton
``dx`` kernel followed by two eager passes for ``dw`` (``rmsnorm.py:117-118``).

Unlike the reference there is no CPU fallback: CPU tensors raise.
"""

from __future__ import annotations

import ctypes

import torch

from packbalance_amd import _native as N

HAS_NATIVE = N.available()
# The reference exports HAS_TRITON ("fused kernels available"); kept as an alias.
HAS_TRITON = HAS_NATIVE

_MAX_N = 65536


def _rows(t: torch.Tensor) -> torch.Tensor:
    t2 = t.reshape(-1, t.shape[-1])
    return t2 if t2.stride(-1) == 1 else t2.contiguous()


class _RMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
        N.require_device(x, weight, op="rmsnorm")
        n = x.shape[-1]
        if weight.dim() != 1 or weight.shape[0] != n:
            raise ValueError(f"rmsnorm: weight shape {tuple(weight.shape)} does not match ({n},)")
        if n > _MAX_N:
            raise RuntimeError("RMSNorm feature dimension is too large for this kernel")
        x2d = _rows(x)
        w = weight.contiguous()
        rows = x2d.shape[0]
        y = torch.empty((rows, n), dtype=x.dtype, device=x.device)
        rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
        N.call(
            "pb_rmsnorm_fwd",
            x2d.data_ptr(), x2d.stride(0), N.dtype_code(x2d),
            w.data_ptr(), N.dtype_code(w),
            y.data_ptr(), y.stride(0),
            rstd.data_ptr(), rows, n, float(eps), N.stream_ptr(x),
        )
        ctx.save_for_backward(x2d, w, rstd)
        ctx.w_dtype = weight.dtype
        return y.reshape(x.shape)

    @staticmethod
    def backward(ctx, dy: torch.Tensor):
        x2d, w, rstd = ctx.saved_tensors
        rows, n = x2d.shape
        dy2d = _rows(dy)
        if dy2d.dtype != x2d.dtype:
            dy2d = dy2d.to(x2d.dtype)
        dx = torch.empty((rows, n), dtype=x2d.dtype, device=x2d.device)
        dw = torch.empty(n, dtype=w.dtype, device=w.device)
        ws_bytes = N.lib().pb_rmsnorm_bwd_workspace_bytes(rows, n)
        ws = torch.empty(max(1, ws_bytes // 4), dtype=torch.float32, device=x2d.device)
        N.call(
            "pb_rmsnorm_bwd",
            dy2d.data_ptr(), dy2d.stride(0),
            x2d.data_ptr(), x2d.stride(0), N.dtype_code(x2d),
            w.data_ptr(), N.dtype_code(w),
            rstd.data_ptr(),
            dx.data_ptr(), dx.stride(0),
            dw.data_ptr(), ws.data_ptr(), rows, n, N.stream_ptr(dx),
        )
        if dx.dtype != dy.dtype:
            dx = dx.to(dy.dtype)
        return dx.reshape(dy.shape), dw.to(ctx.w_dtype), None


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``x * rsqrt(mean(x^2) + eps) * weight`` with fp32 statistics (gfx950 kernel)."""
    return _RMSNorm.apply(x, weight, eps)


# ---------------------------------------------------------------- fused residual add
def _fwd_call(x2d, d2d, h, w, y, rstd, eps):
    rows, n = x2d.shape
    N.call(
        "pb_add_rmsnorm_fwd",
        x2d.data_ptr(), x2d.stride(0), N.dtype_code(x2d),
        d2d.data_ptr() if d2d is not None else None, d2d.stride(0) if d2d is not None else n,
        N.dtype_code(d2d) if d2d is not None else N.dtype_code(x2d),
        h.data_ptr() if h is not None else None, h.stride(0) if h is not None else n,
        w.data_ptr(), N.dtype_code(w),
        y.data_ptr(), y.stride(0), N.dtype_code(y),
        rstd.data_ptr(), rows, n, float(eps), N.stream_ptr(x2d),
    )


def _bwd_call(dy2d, h2d, w, rstd, dres, dx, ddelta, dw, accumulate=False):
    rows, n = h2d.shape
    ws_bytes = N.lib().pb_add_rmsnorm_bwd_workspace_bytes(rows, n)
    ws = torch.empty(max(1, ws_bytes // 4), dtype=torch.float32, device=h2d.device)
    N.call(
        "pb_add_rmsnorm_bwd",
        dy2d.data_ptr(), dy2d.stride(0), N.dtype_code(dy2d),
        h2d.data_ptr(), h2d.stride(0), N.dtype_code(h2d),
        w.data_ptr(), N.dtype_code(w), rstd.data_ptr(),
        dres.data_ptr() if dres is not None else None, dres.stride(0) if dres is not None else n,
        dx.data_ptr(), dx.stride(0),
        ddelta.data_ptr() if ddelta is not None else None,
        ddelta.stride(0) if ddelta is not None else n,
        N.dtype_code(ddelta) if ddelta is not None else N.dtype_code(dx),
        dw.data_ptr(), int(accumulate), ws.data_ptr(), rows, n, N.stream_ptr(h2d),
    )


def _bwd_partials_call(dy2d, h2d, w, rstd, dres, dx, ddelta, partials):
    """The backward without its dw reduction: the per-workgroup fp32 dw partials go
    to ``partials`` (``pb_add_rmsnorm_bwd_workspace_bytes`` bytes) for a later
    batched reduction (``pb_rmsnorm_dw_reduce_batched``)."""
    rows, n = h2d.shape
    N.call(
        "pb_add_rmsnorm_bwd_partials",
        dy2d.data_ptr(), dy2d.stride(0), N.dtype_code(dy2d),
        h2d.data_ptr(), h2d.stride(0), N.dtype_code(h2d),
        w.data_ptr(), N.dtype_code(w), rstd.data_ptr(),
        dres.data_ptr() if dres is not None else None, dres.stride(0) if dres is not None else n,
        dx.data_ptr(), dx.stride(0),
        ddelta.data_ptr() if ddelta is not None else None,
        ddelta.stride(0) if ddelta is not None else n,
        N.dtype_code(ddelta) if ddelta is not None else N.dtype_code(dx),
        partials.data_ptr(), rows, n, N.stream_ptr(h2d),
    )


def partial_floats(rows: int, n: int) -> int:
    """fp32 elements of one norm backward's dw partial table."""
    return N.lib().pb_add_rmsnorm_bwd_workspace_bytes(rows, n) // 4


def dw_reduce_batched(partials: torch.Tensor, dws: list, rows: int, n: int) -> None:
    """dws[i] (fp32 [n]) += the column sums of partials[i] ([count, >= partial_floats])."""
    ptrs = (ctypes.c_void_p * len(dws))(*[g.data_ptr() for g in dws])
    N.call("pb_rmsnorm_dw_reduce_batched", partials.data_ptr(), partials.stride(0), ptrs,
           len(dws), rows, n, N.stream_ptr(partials))


def _check_acc(dw_acc, weight):
    if dw_acc is None:
        return
    if (dw_acc.dtype != torch.float32 or weight.dtype != torch.float32
            or dw_acc.shape != weight.shape or not dw_acc.is_contiguous()):
        raise ValueError("dw_acc must be a contiguous fp32 tensor shaped like an fp32 weight")


def _check(x, weight, op):
    N.require_device(x, weight, op=op)
    n = x.shape[-1]
    if weight.dim() != 1 or weight.shape[0] != n:
        raise ValueError(f"{op}: weight shape {tuple(weight.shape)} does not match ({n},)")
    if n > _MAX_N:
        raise RuntimeError("RMSNorm feature dimension is too large for this kernel")


def _out_buffer(buf, rows, n, dtype, device, what):
    """``buf`` as the [rows, n] output (a caller-provided contiguous buffer), else a new one."""
    if buf is None:
        return torch.empty((rows, n), dtype=dtype, device=device)
    if buf.shape != (rows, n) or buf.dtype != dtype or not buf.is_contiguous():
        raise ValueError(f"{what}: output buffer must be a contiguous {dtype} [{rows}, {n}] tensor")
    return buf


class _AddRMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, delta, weight, eps, out_dtype, dw_acc, y_out, ddelta_out, dw_defer):
        _check(x, weight, "add_rmsnorm")
        _check_acc(dw_acc, weight)
        if delta.shape != x.shape:
            raise ValueError(f"add_rmsnorm: delta {tuple(delta.shape)} and x {tuple(x.shape)} differ")
        x2d, d2d, w = _rows(x), _rows(delta), weight.contiguous()
        rows, n = x2d.shape
        h = torch.empty((rows, n), dtype=x.dtype, device=x.device)
        y = _out_buffer(y_out, rows, n, out_dtype, x.device, "add_rmsnorm(y_out)")
        if ddelta_out is not None:
            _out_buffer(ddelta_out, rows, n, delta.dtype, x.device, "add_rmsnorm(ddelta_out)")
        rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
        _fwd_call(x2d, d2d, h, w, y, rstd, eps)
        ctx.save_for_backward(h, w, rstd)
        ctx.meta = (x.shape, delta.dtype, weight.dtype)
        ctx.dw_acc = dw_acc
        ctx.dw_defer = dw_defer if dw_acc is not None else None
        ctx.ddelta_out = ddelta_out
        return h.reshape(x.shape), y.reshape(x.shape)

    @staticmethod
    def backward(ctx, dh, dy):
        h, w, rstd = ctx.saved_tensors
        shape, delta_dtype, w_dtype = ctx.meta
        rows, n = h.shape
        dy2d = _rows(dy) if dy is not None else torch.zeros_like(h)
        dres = None
        if dh is not None:
            dres = _rows(dh)
            dres = dres if dres.dtype == h.dtype else dres.to(h.dtype)
        dx = torch.empty_like(h)
        ddelta = _out_buffer(ctx.ddelta_out, rows, n, delta_dtype, h.device, "add_rmsnorm")
        if ctx.dw_defer is not None:
            plan, slot = ctx.dw_defer
            _bwd_partials_call(dy2d, h, w, rstd, dres, dx, ddelta, plan.norm_partials(slot))
            plan.add_norm(slot, ctx.dw_acc)
            return (dx.reshape(shape), ddelta.reshape(shape), None, None, None, None, None, None,
                    None)
        if ctx.dw_acc is not None:
            _bwd_call(dy2d, h, w, rstd, dres, dx, ddelta, ctx.dw_acc, accumulate=True)
            return (dx.reshape(shape), ddelta.reshape(shape), None, None, None, None, None, None,
                    None)
        dw = torch.empty(n, dtype=w.dtype, device=w.device)
        _bwd_call(dy2d, h, w, rstd, dres, dx, ddelta, dw)
        return (dx.reshape(shape), ddelta.reshape(shape), dw.to(w_dtype), None, None, None, None,
                None, None)


class _RMSNormTo(torch.autograd.Function):
    """RMSNorm whose output dtype differs from the input's (no residual add)."""

    @staticmethod
    def forward(ctx, x, weight, eps, out_dtype, dw_acc, y_out, dw_defer):
        _check(x, weight, "rmsnorm")
        _check_acc(dw_acc, weight)
        x2d, w = _rows(x), weight.contiguous()
        rows, n = x2d.shape
        y = _out_buffer(y_out, rows, n, out_dtype, x.device, "rmsnorm(y_out)")
        rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
        _fwd_call(x2d, None, None, w, y, rstd, eps)
        ctx.save_for_backward(x2d, w, rstd)
        ctx.meta = (x.shape, weight.dtype)
        ctx.dw_acc = dw_acc
        ctx.dw_defer = dw_defer if dw_acc is not None else None
        return y.reshape(x.shape)

    @staticmethod
    def backward(ctx, dy):
        x2d, w, rstd = ctx.saved_tensors
        shape, w_dtype = ctx.meta
        dx = torch.empty_like(x2d)
        if ctx.dw_defer is not None:
            plan, slot = ctx.dw_defer
            _bwd_partials_call(_rows(dy), x2d, w, rstd, None, dx, None, plan.norm_partials(slot))
            plan.add_norm(slot, ctx.dw_acc)
            return dx.reshape(shape), None, None, None, None, None, None
        if ctx.dw_acc is not None:
            _bwd_call(_rows(dy), x2d, w, rstd, None, dx, None, ctx.dw_acc, accumulate=True)
            return dx.reshape(shape), None, None, None, None, None, None
        dw = torch.empty(x2d.shape[1], dtype=w.dtype, device=w.device)
        _bwd_call(_rows(dy), x2d, w, rstd, None, dx, None, dw)
        return dx.reshape(shape), dw.to(w_dtype), None, None, None, None, None


def add_rmsnorm(x: torch.Tensor, delta: torch.Tensor, weight: torch.Tensor, eps: float,
                out_dtype: torch.dtype | None = None, dw_acc: torch.Tensor | None = None,
                y_out: torch.Tensor | None = None, ddelta_out: torch.Tensor | None = None,
                dw_defer=None):
    """Residual add fused with the next RMSNorm (gfx950 kernel).

    Returns ``(h, y)``: ``h = x + delta`` in x's dtype (the new residual stream) and
    ``y = rmsnorm(h, weight, eps)`` in ``out_dtype`` (default x's dtype).  The backward
    takes the gradients of both outputs and returns them summed into ``dx`` (x's dtype)
    and ``ddelta`` (delta's dtype), so no separate add or cast kernels run.  With
    ``dw_acc`` (fp32, shaped like an fp32 ``weight``) the weight gradient is ADDED to
    ``dw_acc`` by the backward kernel and the gradient returned for ``weight`` is None.
    ``y_out`` / ``ddelta_out`` (contiguous [rows, n] buffers) receive y and the
    backward's ddelta instead of new tensors (the decoder's batched weight-gradient
    plan hands out its slots this way).  ``dw_defer = (plan, slot)`` (with ``dw_acc``)
    leaves the backward's dw partials in ``plan.norm_partials(slot)`` and registers
    ``dw_acc`` with ``plan.add_norm``: the plan reduces every deferred norm of the
    pass in one launch when the backward ends (same bits as the immediate sum).
    """
    return _AddRMSNorm.apply(x, delta, weight, eps, out_dtype or x.dtype, dw_acc, y_out,
                             ddelta_out, dw_defer)


def rmsnorm_to(x: torch.Tensor, weight: torch.Tensor, eps: float,
               out_dtype: torch.dtype, dw_acc: torch.Tensor | None = None,
               y_out: torch.Tensor | None = None, dw_defer=None) -> torch.Tensor:
    """``rmsnorm`` written directly in ``out_dtype`` (e.g. fp32 residual -> bf16 activations);
    ``dw_acc``, ``y_out`` and ``dw_defer`` as for ``add_rmsnorm``."""
    if out_dtype == x.dtype and dw_acc is None and y_out is None:
        return rmsnorm(x, weight, eps)
    return _RMSNormTo.apply(x, weight, eps, out_dtype, dw_acc, y_out, dw_defer)
