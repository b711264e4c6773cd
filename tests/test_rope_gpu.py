"""GPU parity: fused RoPE (q and k in one launch) vs the oracle.

The kernel rotates each (d, d + D/2) pair in fp32 and rounds once to the
tensor dtype, so against the float64 oracle on the same stored inputs the
error is one rounding: bf16 within 1 ulp (relative 2^-7), fp32 within 1e-6
relative.  The reference (rope.py:38-41) rounds cos/sin, both products and
the sum to bf16; the kernel stays within 3 half-ulps of the products' size of
that sequence.
Backward: the incoming gradients rotated by -theta (the adjoint, pinned in
the oracle tests).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kernels as OK
from packbalance_amd.data import workloads as W
from packbalance_amd.model.rope import RotaryEmbedding, apply_rotary_pos_emb, rotate_half

pytestmark = pytest.mark.gpu

RTOL = {torch.bfloat16: 2.0 ** -7, torch.float32: 1e-6}


def _qk(B, Hq, Hkv, S, D, dtype, dev, model_layout, seed=0):
    g = torch.Generator().manual_seed(seed)
    if model_layout:  # .transpose(1, 2) views of [B, S, H, D], as the model makes them
        q = torch.randn(B, S, Hq, D, generator=g).to(dev, dtype).transpose(1, 2)
        k = torch.randn(B, S, Hkv, D, generator=g).to(dev, dtype).transpose(1, 2)
    else:
        q = torch.randn(B, Hq, S, D, generator=g).to(dev, dtype)
        k = torch.randn(B, Hkv, S, D, generator=g).to(dev, dtype)
    return q, k


def _cos_sin(B, S, D, dev):
    """cos/sin gathered by per-document position ids (packed documents)."""
    packs = [[S // 3, S // 4, S - S // 3 - S // 4]] * B
    batch = W.pack_tensors(packs, S, 100, np.random.default_rng(0))
    rot = RotaryEmbedding(D, S).to(dev)
    return rot(batch.position_ids.to(dev))


def _close(got, want, dtype, what):
    torch.testing.assert_close(got.detach().double().cpu(), want, rtol=RTOL[dtype], atol=1e-6,
                               msg=lambda m: f"{what}: {m}")


@pytest.mark.parametrize(
    "B,Hq,Hkv,S,D,dtype,model_layout",
    [
        (1, 12, 4, 2048, 64, torch.bfloat16, True),  # cfg2 attention shape
        (2, 4, 2, 256, 32, torch.bfloat16, True),  # cfg1 shape
        (2, 8, 2, 300, 128, torch.bfloat16, False),
        (1, 4, 4, 64, 64, torch.float32, True),
        (2, 3, 1, 40, 6, torch.bfloat16, True),  # half-dim 3: scalar path
    ],
)
def test_rope_forward_backward_match_oracle(B, Hq, Hkv, S, D, dtype, model_layout, dev) -> None:
    q, k = _qk(B, Hq, Hkv, S, D, dtype, dev, model_layout)
    cos, sin = _cos_sin(B, S, D, dev)
    qr, kr = q.detach().requires_grad_(True), k.detach().requires_grad_(True)
    qo, ko = apply_rotary_pos_emb(qr, kr, cos, sin)
    assert qo.dtype == dtype and qo.shape == q.shape and qo.stride() == q.stride()
    _close(qo, OK.rope(q, cos, sin), dtype, "q out")
    _close(ko, OK.rope(k, cos, sin), dtype, "k out")
    gq, gk = _qk(B, Hq, Hkv, S, D, dtype, dev, model_layout, seed=1)
    torch.autograd.backward((qo, ko), (gq, gk))
    _close(qr.grad, OK.rope(gq, cos, sin, inverse=True), dtype, "dq")
    _close(kr.grad, OK.rope(gk, cos, sin, inverse=True), dtype, "dk")


def test_rope_within_three_ulps_of_the_reference_bf16_sequence(dev) -> None:
    """rope.py:38-41 computed as the reference does (every op rounded to bf16)."""
    q, k = _qk(1, 8, 2, 512, 64, torch.bfloat16, dev, True, seed=4)
    cos, sin = _cos_sin(1, 512, 64, dev)
    c = torch.cat((cos, cos), dim=-1).unsqueeze(1).to(torch.bfloat16)
    s = torch.cat((sin, sin), dim=-1).unsqueeze(1).to(torch.bfloat16)
    ref_q = (q * c) + (rotate_half(q) * s)
    qo, _ = apply_rotary_pos_emb(q, k, cos, sin)
    # The reference rounds cos/sin, each product and the sum: its error scales
    # with the size of the products, not of their (possibly cancelling) sum.
    terms = (q.float() * c.float()).abs() + (rotate_half(q).float() * s.float()).abs()
    err = (qo.float() - ref_q.float()).abs()
    assert bool((err <= 3 * 2.0 ** -8 * terms + 1e-6).all()), float((err / (terms + 1e-6)).max())


def test_rope_broadcast_cos_and_errors(dev) -> None:
    q, k = _qk(2, 4, 2, 64, 32, torch.bfloat16, dev, True)
    cos, sin = _cos_sin(1, 64, 32, dev)  # [1, S, D/2] broadcast over the batch
    qo, ko = apply_rotary_pos_emb(q, k, cos, sin)
    _close(qo, OK.rope(q, cos.expand(2, -1, -1), sin.expand(2, -1, -1)), torch.bfloat16, "q out")
    with pytest.raises(ValueError):
        apply_rotary_pos_emb(q, k, cos[:, :10], sin[:, :10])
    with pytest.raises(RuntimeError):
        apply_rotary_pos_emb(q.cpu(), k.cpu(), cos.cpu(), sin.cpu())
