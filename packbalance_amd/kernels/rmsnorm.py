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
