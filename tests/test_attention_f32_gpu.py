"""GPU parity: fp32 document-masked GQA attention (the reference's non-autocast path).

fp32 q/k/v run the fp32 kernels (the reference's FlexAttention computes fp32
tensors in fp32, packbalance/model/attention.py:116-122); outputs and
gradients against the float64 oracle on the same fp32 inputs at fp32-level
tolerances: elementwise 2e-5 absolute + 2e-4 relative, and 1e-5 in relative
Frobenius norm.  fp16 inputs are widened to fp32 and the result rounded to
fp16 (checked at fp16's own rounding).  Padding rows (doc_id -1) follow
FlexAttention's mask_mod (a pad attends to earlier pads).
"""

from __future__ import annotations

import pytest
import torch

from oracle import attention as OA
from packbalance_amd.data import workloads as W
from packbalance_amd.model.attention import doc_attention

pytestmark = pytest.mark.gpu


def _rel_fro(got, want):
    g, w = got.detach().double().cpu(), want.double()
    return float((g - w).norm() / w.norm().clamp_min(1e-30))


def _inputs(B, Hq, Hkv, S, D, dev, dtype=torch.float32, *, seed=0, model_layout=True):
    g = torch.Generator().manual_seed(seed)
    shp = (lambda H: (B, S, H, D)) if model_layout else (lambda H: (B, H, S, D))
    out = []
    for H in (Hq, Hkv, Hkv, Hq):
        t = torch.randn(*shp(H), generator=g).to(dev, dtype)
        out.append(t.transpose(1, 2) if model_layout else t)
    return out


def _check(q, k, v, do, doc, what, *, scale=None, atol=2e-5, rtol=2e-4, fro=1e-5):
    qr, kr, vr = (t.detach().requires_grad_(True) for t in (q, k, v))
    out = doc_attention(qr, kr, vr, doc, scale=scale)
    out.backward(do)
    assert out.dtype == q.dtype and out.shape == q.shape
    ref = OA.attention(q, k, v, doc.cpu(), do, **({} if scale is None else {"scale": scale}))
    for got, name in ((out, "out"), (qr.grad, "dq"), (kr.grad, "dk"), (vr.grad, "dv")):
        assert got.dtype == q.dtype, name
        torch.testing.assert_close(got.detach().double().cpu(), ref[name].double(), atol=atol,
                                   rtol=rtol, msg=lambda m, n=name: f"{what} {n}: {m}")
        assert _rel_fro(got, ref[name]) < fro, (what, name, _rel_fro(got, ref[name]))


@pytest.mark.parametrize(
    "B,Hq,Hkv,S,D,docs",
    [
        (1, 2, 2, 64, 16, [20, 44]),  # the reference's flex test shape
        (1, 4, 2, 256, 32, [60, 50, 100, 46]),  # cfg1 shape
        (2, 4, 1, 300, 64, [100, 150, -50]),  # -n: n pad tokens (doc -1)
        (1, 6, 2, 200, 128, [1] * 50 + [150]),  # single-token documents, D 128
        (3, 4, 4, 130, 30, [64, 66]),  # D % 4 != 0 (scalar row reads)
        (1, 8, 2, 257, 100, [257]),  # one dense document, odd S
        (1, 12, 4, 2048, 64, "cfg2"),  # cfg2 shape, heavy-tail pack
    ],
)
def test_f32_attention_matches_oracle(B, Hq, Hkv, S, D, docs, dev) -> None:
    if docs == "cfg2":
        packs = W.cfg2_steps(1)[0][:B]
    else:
        pad = sum(-d for d in docs if d < 0)
        packs = [[d for d in docs if d > 0]] * B
        assert sum(packs[0]) + pad == S
    doc = W.doc_ids_from_lengths(packs, S).to(dev)
    q, k, v, do = _inputs(B, Hq, Hkv, S, D, dev, seed=S + D)
    _check(q, k, v, do, doc, f"B{B} Hq{Hq} Hkv{Hkv} S{S} D{D}")


def test_f32_attention_noncontiguous_documents_and_layout(dev) -> None:
    """Document ids that recur in several runs (the mask compares ids), on contiguous
    [B, H, S, D] tensors, with a non-default scale."""
    S = 160
    ids = torch.tensor([i % 3 for i in range(S)], device=dev)[None]
    q, k, v, do = _inputs(1, 4, 2, S, 32, dev, seed=7, model_layout=False)
    _check(q, k, v, do, ids, "alternating docs", scale=0.3)


def test_f16_attention_is_computed_in_fp32(dev) -> None:
    """fp16 q/k/v: widened, computed in fp32, returned in fp16 -- within fp16's rounding
    of the float64 result (relative 2^-10)."""
    q, k, v, do = _inputs(1, 4, 2, 256, 64, dev, torch.float16, seed=3)
    doc = W.doc_ids_from_lengths([[100, 156]], 256).to(dev)
    _check(q, k, v, do, doc, "fp16", atol=2e-3, rtol=2e-3, fro=1e-3)


def test_f32_attention_empty_grad_paths(dev) -> None:
    """Only the output used: gradients of q/k/v still come out (zeros through a zero dO)."""
    q, k, v, _ = _inputs(1, 2, 1, 64, 16, dev, seed=11)
    doc = W.doc_ids_from_lengths([[30, 34]], 64).to(dev)
    qr, kr, vr = (t.detach().requires_grad_(True) for t in (q, k, v))
    out = doc_attention(qr, kr, vr, doc)
    (out * 0).sum().backward()
    for g in (qr.grad, kr.grad, vr.grad):
        assert g is not None and float(g.abs().max()) == 0.0


def test_f32_backward_chunked_walks_repeat_bit_for_bit(dev) -> None:
    """Small grids cut the dK/dV walk (heads x query sub-tiles) into chunks whose fp32
    partials are summed in chunk order: two backward passes give identical bits, and the
    workspace holds more than delta exactly when the grid is split."""
    from packbalance_amd import _native as N

    B, Hq, Hkv, S, D = 1, 12, 4, 2048, 64
    packs = W.cfg2_steps(1)[0][:B]
    doc = W.doc_ids_from_lengths(packs, S).to(dev)
    q, k, v, do = _inputs(B, Hq, Hkv, S, D, dev, seed=21)
    delta_bytes = B * Hq * S * 4
    assert N.lib().pb_attn_bwd_f32_workspace_bytes(B, Hq, Hkv, S, D) > delta_bytes
    # 8 packs x 8 KV heads x 64 KV tiles = 4096 tiles: no split, delta only
    assert N.lib().pb_attn_bwd_f32_workspace_bytes(8, 32, 8, 8192, 128) == 8 * 32 * 8192 * 4
    grads = []
    for _ in range(2):
        qr, kr, vr = (t.detach().requires_grad_(True) for t in (q, k, v))
        doc_attention(qr, kr, vr, doc).backward(do)
        torch.cuda.synchronize()
        grads.append((qr.grad.clone(), kr.grad.clone(), vr.grad.clone()))
    for a, b in zip(*grads):
        assert torch.equal(a, b)
