"""Fused SwiGLU on the gfx950 kernels of ``libpackbalance_amd.so``.

Same public API as the reference ``packbalance/kernels/swiglu.py:72-75``
(``swiglu(gate, up)``) and the autograd contract of ``_SwiGLU``
(``swiglu.py:49-69``): saves ``(gate, up)``, output in the gate dtype, fp32
math.  Unlike the reference there is no CPU fallback: CPU tensors raise.
"""

from __future__ import annotations

import torch

from packbalance_amd import _native as N

HAS_NATIVE = N.available()
HAS_TRITON = HAS_NATIVE


class _SwiGLU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
        N.require_device(gate, up, op="swiglu")
        if gate.shape != up.shape:
            raise ValueError(f"swiglu: gate {tuple(gate.shape)} and up {tuple(up.shape)} differ")
        g = gate.contiguous()
        u = up.contiguous() if up.dtype == gate.dtype else up.to(gate.dtype).contiguous()
        out = torch.empty_like(g)
        N.call("pb_swiglu_fwd", g.data_ptr(), u.data_ptr(), out.data_ptr(), g.numel(),
               N.dtype_code(g), N.stream_ptr(g))
        ctx.save_for_backward(g, u)
        ctx.up_dtype = up.dtype
        return out

    @staticmethod
    def backward(ctx, dy: torch.Tensor):
        g, u = ctx.saved_tensors
        d = dy.contiguous() if dy.dtype == g.dtype else dy.to(g.dtype).contiguous()
        dg = torch.empty_like(g)
        du = torch.empty_like(u)
        N.call("pb_swiglu_bwd", g.data_ptr(), u.data_ptr(), d.data_ptr(), dg.data_ptr(),
               du.data_ptr(), g.numel(), N.dtype_code(g), N.stream_ptr(g))
        return dg, du.to(ctx.up_dtype)


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``silu(gate) * up`` (gfx950 kernel)."""
    return _SwiGLU.apply(gate, up)
