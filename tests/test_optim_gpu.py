"""GPU parity: the fused clip + AdamW step over a flat store.

Checked against the float64 oracle (``oracle/optim.py``, itself pinned to
torch's clip_grad_norm_ + AdamW) on the same fp32 inputs over several steps,
with clipping active on some steps and not on others: parameters, moments
and the gradient norm within fp32 rounding -- the norm and moments to rtol
2e-6 (moments with an absolute floor of 1e-6 of their largest entry, for
entries that cancel towards zero), parameters to one fp32 ulp of the largest
parameter per step taken plus 1e-5 of the learning rate (an update computed
wrongly is off by ~lr).  The bf16 weight copy must equal
the updated fp32 parameters rounded to bf16, bit for bit.  A second check
compares against torch's own fused AdamW on the GPU.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import optim as OO
from packbalance_amd.model.flat import FlatParams
from packbalance_amd.model.optim import FlatAdamW

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)


def _store(n_each, dev, seed=0):
    g = torch.Generator().manual_seed(seed)
    mod = torch.nn.Module()
    for i, n in enumerate(n_each):
        mod.register_parameter(f"p{i}", torch.nn.Parameter(torch.randn(n, generator=g) * 0.02))
    return FlatParams(mod.to(dev))


@pytest.mark.parametrize("max_norm", [1.0, 0.0])
def test_flat_adamw_matches_oracle(max_norm, dev) -> None:
    flat = _store([1000003, 517, 64 * 64], dev)  # odd sizes: vector tails and padding
    n = flat.master.numel()
    opt = FlatAdamW(flat, max_grad_norm=max_norm, copy_dtype=torch.bfloat16, **HP)
    p = flat.master.double().cpu().numpy().copy()
    m, v = np.zeros(n), np.zeros(n)
    step = 0
    rng = np.random.default_rng(1)
    for k in range(4):
        g = (rng.standard_normal(n) * (0.002 if k % 2 else 0.05)).astype(np.float32)
        flat.grad.copy_(torch.from_numpy(g))
        norm = opt.step()
        step, onorm = OO.clip_adamw_step(p, g.astype(np.float64), m, v, step, max_norm=max_norm,
                                         **HP)
        torch.cuda.synchronize()
        assert int(opt.step_count.item()) == step
        assert abs(float(norm) - onorm) <= 2e-6 * onorm
        got_p = flat.master.double().cpu().numpy()
        err = np.abs(got_p - p).max()
        ulp = float(np.spacing(np.float32(np.abs(p).max())))
        assert err <= (k + 1) * ulp + 1e-5 * HP["lr"], (k, err, ulp)
        np.testing.assert_allclose(opt.exp_avg.double().cpu().numpy(), m, rtol=2e-6,
                                   atol=1e-6 * np.abs(m).max())
        np.testing.assert_allclose(opt.exp_avg_sq.double().cpu().numpy(), v, rtol=2e-6,
                                   atol=1e-6 * np.abs(v).max())
        shadow = flat.weight([p_ for p_ in flat._params[:1]], torch.bfloat16)
        assert torch.equal(shadow, flat._params[0].detach().to(torch.bfloat16))
    # The grad buffer is read, not written.
    assert torch.equal(flat.grad.cpu(), torch.from_numpy(g))


def test_flat_adamw_matches_torch_fused_adamw(dev) -> None:
    flat = _store([4096 * 768, 33], dev, seed=2)
    ref = torch.nn.Parameter(flat.master.detach().clone())
    topt = torch.optim.AdamW([ref], fused=True, **HP)
    opt = FlatAdamW(flat, max_grad_norm=1.0, **HP)
    g0 = torch.Generator(device=dev).manual_seed(3)
    for k in range(3):
        g = torch.randn(flat.master.numel(), device=dev, generator=g0) * (0.05 if k else 0.001)
        flat.grad.copy_(g)
        ref.grad = g.clone()
        tn = torch.nn.utils.clip_grad_norm_([ref], 1.0)
        topt.step()
        norm = opt.step()
        torch.testing.assert_close(norm, tn, rtol=2e-6, atol=0)
        # a few fp32 ulps of the largest parameter (~0.1), far below one update (~lr)
        torch.testing.assert_close(flat.master, ref.detach(), rtol=0, atol=4e-8)


def test_flat_adamw_sums_gradient_slots(dev) -> None:
    """Three gradient slots: the step uses their sum (slot order 0, 1, 2 in fp32),
    leaves it in slot 0 bit for bit, and otherwise matches the oracle on that sum."""
    g = torch.Generator().manual_seed(5)
    mod = torch.nn.Module()
    mod.register_parameter("a", torch.nn.Parameter(torch.randn(300007, generator=g) * 0.02))
    mod.register_parameter("b", torch.nn.Parameter(torch.randn(77, generator=g) * 0.02))
    flat = FlatParams(mod.to(dev), grad_slots=3)
    assert flat.grad_slots == 3 and flat.grad_slot_stride >= flat.master.numel()
    n = flat.master.numel()
    opt = FlatAdamW(flat, max_grad_norm=1.0, copy_dtype=torch.bfloat16, **HP)
    p = flat.master.double().cpu().numpy().copy()
    m, v = np.zeros(n), np.zeros(n)
    step = 0
    rng = np.random.default_rng(6)
    for k in range(2):
        parts = [(rng.standard_normal(n) * 0.01).astype(np.float32) for _ in range(3)]
        for s, part in enumerate(parts):
            flat._grads[s].copy_(torch.from_numpy(part))
        total = (parts[0] + parts[1]) + parts[2]  # fp32, in slot order
        norm = opt.step()
        step, onorm = OO.clip_adamw_step(p, total.astype(np.float64), m, v, step, max_norm=1.0,
                                         **HP)
        torch.cuda.synchronize()
        assert np.array_equal(flat.grad.cpu().numpy(), total)
        assert abs(float(norm) - onorm) <= 2e-6 * onorm
        ulp = float(np.spacing(np.float32(np.abs(p).max())))
        assert np.abs(flat.master.double().cpu().numpy() - p).max() <= (k + 1) * ulp + 1e-5 * HP["lr"]
    with flat.accumulate_into(2):
        assert flat.grad_of([mod.b]).data_ptr() == flat._grads[2].data_ptr() + \
            (mod.b.data_ptr() - flat.master.data_ptr())
    with pytest.raises(ValueError):
        with flat.accumulate_into(3):
            pass


def test_flat_adamw_rejects_bad_hyperparameters(dev) -> None:
    flat = _store([64], dev)
    with pytest.raises(ValueError):
        FlatAdamW(flat, betas=(1.0, 0.9))
