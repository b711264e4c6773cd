"""Clip-by-global-norm + AdamW as one fused step over a ``FlatParams`` store.

The reference's train loop (``packbalance/train/train.py:58-69,353-362``,
``profiling/bench_train.py:79-85,115-116``) calls
``torch.nn.utils.clip_grad_norm_(model.parameters(), clip)`` and then a fused
``torch.optim.AdamW(model.parameters(), lr, betas, weight_decay).step()``.
With uniform hyper-parameters both are element-wise over the parameter set,
so over the flat store they are three launches of ``pb_clip_adamw_step``
(gradient norm partials, a one-workgroup fold that also advances the
device-resident step count, the element-wise update), and the update writes
the bf16 copy the next step's matmuls read.  The step count, the norm and the
per-step scalars stay on the device (graph-capture safe).  When the store
holds several gradient slots (micro-batches run concurrently), the norm pass
first sums them into slot 0, so ``.grad`` ends the step holding the whole
step's gradient.  Unlike ``clip_grad_norm_``, the clipped gradient is not
written back into ``.grad``.
"""

from __future__ import annotations

import torch

from packbalance_amd import _native as N
from packbalance_amd.model.flat import FlatParams


class FlatAdamW:
    def __init__(self, flat: FlatParams, lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 1e-2, max_grad_norm: float = 0.0,
                 copy_dtype: torch.dtype | None = None) -> None:
        if not (0.0 <= betas[0] < 1.0 and 0.0 <= betas[1] < 1.0 and eps > 0.0):
            raise ValueError(f"bad AdamW hyper-parameters betas={betas} eps={eps}")
        self.flat = flat
        self.lr, self.betas, self.eps = float(lr), (float(betas[0]), float(betas[1])), float(eps)
        self.weight_decay, self.max_grad_norm = float(weight_decay), float(max_grad_norm)
        self.copy_dtype = copy_dtype if copy_dtype not in (None, torch.float32) else None
        dev = flat.master.device
        n = flat.master.numel()
        self.exp_avg = torch.zeros(n, dtype=torch.float32, device=dev)
        self.exp_avg_sq = torch.zeros(n, dtype=torch.float32, device=dev)
        self.step_count = torch.zeros(1, dtype=torch.float32, device=dev)
        self.grad_norm = torch.zeros(1, dtype=torch.float32, device=dev)
        ws = N.lib().pb_clip_adamw_workspace_bytes(n)
        self._ws = torch.empty((ws + 15) // 16 * 4, dtype=torch.float32, device=dev)

    def step(self) -> torch.Tensor:
        """Clip and update; returns the pre-clip gradient norm (device scalar)."""
        f = self.flat
        copy = None
        if self.copy_dtype is not None:
            copy = f._shadow_buf(self.copy_dtype)
        N.call("pb_clip_adamw_step", f.master.data_ptr(), f.grad.data_ptr(), f.grad_slots,
               f.grad_slot_stride, self.exp_avg.data_ptr(), self.exp_avg_sq.data_ptr(),
               copy.data_ptr() if copy is not None else None,
               N.dtype_code(copy) if copy is not None else N.PB_F32, f.master.numel(),
               self.lr, self.betas[0], self.betas[1], self.eps, self.weight_decay,
               self.max_grad_norm, self.step_count.data_ptr(), self.grad_norm.data_ptr(),
               self._ws.data_ptr(), N.stream_ptr(f.master))
        if copy is not None:
            f.mark_fresh(self.copy_dtype)
        return self.grad_norm[0]
