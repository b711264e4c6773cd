"""Cross-entropy kernels on gfx950: the row CE over materialised logits.

``ce_rows`` is the contract of the reference's ``_ce_launch`` / ``_ce_kernel``
(``packbalance/kernels/fused_ce.py:31-118``): per-row loss (and optionally
dlogits) over a ``[M, V]`` logits block with any strides.
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
            ignore_index: int = -100, z_loss_coeff: float = 0.0):
    """Per-row CE of a logits block: returns (loss fp32 [M], lse fp32 [M], dlogits | None).

    dlogits has the dtype and strides of ``logits`` (``torch.empty_like``).
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
    if write_dlogits:
        dl = torch.empty_like(logits)
        if dl.stride() != logits.stride():  # non-dense view: the kernel shares strides
            logits = logits.contiguous()
            dl = torch.empty_like(logits)
    loss = torch.empty(m, dtype=torch.float32, device=logits.device)
    lse = torch.empty(m, dtype=torch.float32, device=logits.device)
    N.call(
        "pb_ce_rows",
        logits.data_ptr(), logits.stride(0), logits.stride(1), N.dtype_code(logits),
        t.data_ptr(), loss.data_ptr(), lse.data_ptr(), N.ptr(dl),
        m, v, int(ignore_index), float(z_loss_coeff), N.stream_ptr(logits),
    )
    return loss, lse, dl
