"""CPU restatement of the reference's optimizer step (test oracle).

The reference's train loop (``packbalance/train/train.py:58-69,353-362``;
``profiling/bench_train.py:79-85,115-116``) calls
``torch.nn.utils.clip_grad_norm_(params, max_norm)`` and then
``torch.optim.AdamW(params, lr, betas, eps, weight_decay, fused=True).step()``.
Both live in PyTorch (pinned here at the image's torch 2.10); this is their
published algorithm -- gradient clipping by global L2 norm, then AdamW
(Loshchilov & Hutter, decoupled weight decay) with PyTorch's bias-correction
form -- in float64 over one flat parameter vector.  ``tests/test_oracle.py``
pins it against ``torch.optim.AdamW`` and ``clip_grad_norm_`` themselves.
"""

from __future__ import annotations

import numpy as np


def clip_adamw_step(p, g, m, v, step: int, *, lr: float, betas, eps: float,
                    weight_decay: float, max_norm: float):
    """One clip + AdamW step.  Arrays are float64 and updated in place
    (p, m, v); returns (new step count, pre-clip gradient norm).

    norm = ||g||_2; c = min(max_norm / (norm + 1e-6), 1) (clip_grad_norm_, with
    c = 1 when max_norm <= 0); t = step + 1; g' = c g;
    p -= lr*wd*p; m = b1 m + (1-b1) g'; v = b2 v + (1-b2) g'^2;
    p -= lr/(1-b1^t) * m / (sqrt(v)/sqrt(1-b2^t) + eps).
    """
    b1, b2 = betas
    norm = float(np.sqrt(np.sum(g * g)))
    c = min(max_norm / (norm + 1e-6), 1.0) if max_norm > 0 else 1.0
    t = step + 1
    gc = g * c
    p -= lr * weight_decay * p
    m *= b1
    m += (1.0 - b1) * gc
    v *= b2
    v += (1.0 - b2) * gc * gc
    denom = np.sqrt(v) / np.sqrt(1.0 - b2 ** t) + eps
    p -= (lr / (1.0 - b1 ** t)) * m / denom
    return t, norm
