"""GPU parity: document-masked GQA attention forward and backward vs the oracle.

Tolerance: outputs and gradients within 2e-2 absolute (plus 2e-2 relative for
entries above 1, where bf16 storage itself rounds by more than 2e-2), bf16
operands with fp32 accumulation, against the float64 oracle on the same
bf16 inputs.  Padding rows (doc_id -1) follow FlexAttention's mask_mod
semantics (a pad attends to earlier pads); the eager convention (pad rows 0)
is checked separately on real rows.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from packbalance_amd.data import workloads as W
from packbalance_amd.model.attention import (
    attention_forward,
    build_doc_block_mask,
    doc_attention,
    flex_attention,
)

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _close(got, want, what):
    torch.testing.assert_close(got.detach().float().cpu(), want.float(), atol=TOL, rtol=TOL,
                               msg=lambda m: f"{what}: {m}")


def _inputs(B, Hq, Hkv, S, D, dev, *, seed=0, model_layout=True):
    """q/k/v as the model makes them: .transpose(1, 2) views of [B, S, H, D] memory."""
    g = torch.Generator().manual_seed(seed)
    if model_layout:
        q = torch.randn(B, S, Hq, D, generator=g).to(dev, torch.bfloat16).transpose(1, 2)
        k = torch.randn(B, S, Hkv, D, generator=g).to(dev, torch.bfloat16).transpose(1, 2)
        v = torch.randn(B, S, Hkv, D, generator=g).to(dev, torch.bfloat16).transpose(1, 2)
        do = torch.randn(B, S, Hq, D, generator=g).to(dev, torch.bfloat16).transpose(1, 2)
    else:
        q = torch.randn(B, Hq, S, D, generator=g).to(dev, torch.bfloat16)
        k = torch.randn(B, Hkv, S, D, generator=g).to(dev, torch.bfloat16)
        v = torch.randn(B, Hkv, S, D, generator=g).to(dev, torch.bfloat16)
        do = torch.randn(B, Hq, S, D, generator=g).to(dev, torch.bfloat16)
    return q, k, v, do


def _run(q, k, v, do, doc, **kw):
    qr, kr, vr = (t.detach().requires_grad_(True) for t in (q, k, v))
    out = doc_attention(qr, kr, vr, doc, **kw)
    out.backward(do)
    return out, qr.grad, kr.grad, vr.grad


def _check(q, k, v, do, doc, what, **kw):
    out, dq, dk, dv = _run(q, k, v, do, doc, **kw)
    ref = OA.attention(q, k, v, doc.cpu(), do)
    _close(out, ref["out"], f"{what} out")
    _close(dq, ref["dq"], f"{what} dq")
    _close(dk, ref["dk"], f"{what} dk")
    _close(dv, ref["dv"], f"{what} dv")


def test_reference_flex_test_case(dev) -> None:
    """tests/test_attention.py:58-73 of the reference: fp32 q/k/v [1,2,64,16]."""
    torch.manual_seed(0)
    q = torch.randn(1, 2, 64, 16, device=dev)
    k = torch.randn(1, 2, 64, 16, device=dev)
    v = torch.randn(1, 2, 64, 16, device=dev)
    doc_ids = torch.tensor([[0] * 20 + [1] * 44], device=dev)
    mask = build_doc_block_mask(doc_ids, n_heads=2)
    out = flex_attention(q, k, v, block_mask=mask)
    assert out.dtype == torch.float32 and out.shape == q.shape
    ref = OA.attention(q, k, v, doc_ids.cpu(), semantics="eager")["out"]
    # fp32 inputs run the fp32 kernels (the reference computes fp32 tensors in fp32)
    torch.testing.assert_close(out.cpu().double(), ref, atol=2e-5, rtol=2e-4)


@pytest.mark.parametrize(
    "B,Hq,Hkv,S,D,docs",
    [
        (1, 2, 2, 64, 16, [20, 44]),
        (1, 4, 2, 256, 32, [60, 50, 100, 46]),  # cfg1 shape
        (2, 4, 1, 300, 64, [100, 150, -50]),  # -n: n pad tokens (doc -1)
        (1, 12, 4, 2048, 64, "cfg2"),  # cfg2 shape, heavy-tail pack
        (1, 8, 8, 1000, 128, [1000]),  # one dense doc, S not a tile multiple
        (1, 6, 2, 200, 128, [1] * 50 + [150]),  # single-token documents
        (3, 4, 4, 130, 100, [64, 66]),  # head dim not a multiple of 16
        (1, 4, 2, 130, 100, [64, 66]),  # split dK/dV, element-wise reduce (D % 8 != 0)
        (1, 8, 2, 1024, 128, [300, 1, 400, -323]),  # pipelined path, 32 query rows per wave
        (2, 16, 4, 2048, 64, "cfg2"),  # pipelined path, 64 query rows per wave, D 64
        # head-split dK/dV with KV lists of >= 16 steps (kKvChunkSteps) walked
        # as two halves:
        (1, 12, 4, 2048, 64, [2048]),  # one dense document (64-step lists)
        (1, 8, 2, 2048, 128, [1100, -948]),  # D 128, a long document then padding
        (2, 6, 2, 1536, 64, [1000, 536]),  # two packs, both documents over the threshold
        # the threshold itself: the 512-token document's first KV tile has a
        # 16-step list (two halves), every other tile 14 steps or fewer (whole)
        (1, 8, 2, 1024, 64, [512, 448, -64]),
        (1, 8, 2, 1024, 128, [512, 448, -64]),
    ],
)
def test_attention_matches_oracle(B, Hq, Hkv, S, D, docs, dev) -> None:
    if docs == "cfg2":
        packs = W.cfg2_steps(1)[0][:B]
    else:
        pad = sum(-d for d in docs if d < 0)
        packs = [[d for d in docs if d > 0]] * B
        assert sum(packs[0]) + pad == S
    doc = W.doc_ids_from_lengths(packs, S).to(dev)
    q, k, v, do = _inputs(B, Hq, Hkv, S, D, dev, seed=S + D)
    _check(q, k, v, do, doc, f"B{B} Hq{Hq} Hkv{Hkv} S{S} D{D}")


def test_attention_contiguous_layout_and_scale(dev) -> None:
    """Contiguous [B, H, S, D] views and a non-default scale (0.3 = 2.4x 1/sqrt(64)).

    The gradients grow with the scale (dQ, dK carry it as a factor and P gets
    sharper), and their error is dominated by the bf16 rounding of O entering
    D = rowsum(dO * O) -- present in any bf16-output implementation -- so the
    absolute gradient tolerance is scaled by scale * sqrt(D) = 2.4 here.
    """
    q, k, v, do = _inputs(1, 4, 2, 192, 64, dev, model_layout=False)
    doc = W.doc_ids_from_lengths([[70, 122]], 192).to(dev)
    out, dq, dk, dv = _run(q, k, v, do, doc, scale=0.3)
    ref = OA.attention(q, k, v, doc.cpu(), do, scale=0.3)
    _close(out, ref["out"], "out")
    # The north star's 2e-2 bar, against the oracle whose delta is formed
    # from the stored bf16 output (as the reference's own backward forms it).
    stored = OA.attention(q, k, v, doc.cpu(), do, scale=0.3, delta_out=out.detach().cpu())
    for got, name in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        _close(got, stored[name], f"{name} (delta from the stored output)")
    gtol = TOL * 0.3 * math.sqrt(64)
    for got, name in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        torch.testing.assert_close(got.detach().float().cpu(), ref[name].float(), atol=gtol,
                                   rtol=TOL, msg=lambda m, n=name: f"{n}: {m}")


def test_attention_noncontiguous_documents(dev) -> None:
    """A document id may appear in several runs: the mask compares ids, not ranges."""
    S = 160
    ids = torch.tensor([i % 3 for i in range(S)], device=dev)[None]
    q, k, v, do = _inputs(1, 2, 1, S, 32, dev, seed=7)
    _check(q, k, v, do, ids, "alternating docs")


def test_attention_noncontiguous_documents_pipelined(dev) -> None:
    """Same, at a shape the DMA-pipelined forward takes (S % 64 == 0, D 64)."""
    S = 256
    ids = torch.tensor([(i // 7) % 3 for i in range(S)], device=dev)[None]
    q, k, v, do = _inputs(1, 4, 2, S, 64, dev, seed=9)
    _check(q, k, v, do, ids, "alternating docs, pipelined")


def test_attention_forward_dispatch_and_eager_rows(dev) -> None:
    packs = [[90, 100]]
    S = 200  # 10 pad tokens
    doc = W.doc_ids_from_lengths(packs, S).to(dev)
    q, k, v, _ = _inputs(1, 4, 2, S, 64, dev, seed=3)
    bm = build_doc_block_mask(doc, 4)
    out = attention_forward(q, k, v, doc, block_mask=bm)
    eager = OA.attention(q, k, v, doc.cpu(), semantics="eager")["out"]
    real = doc[0].cpu() >= 0
    _close(out[:, :, real], eager[:, :, real], "real rows vs eager semantics")
    with pytest.raises(ValueError):
        attention_forward(q, k, v, doc, backend="nope")
    with pytest.raises(RuntimeError):
        attention_forward(q.cpu(), k.cpu(), v.cpu(), doc.cpu())
    with pytest.raises(RuntimeError, match="eager_attention"):
        attention_forward(q, k, v, doc, backend="eager")


def test_attention_deterministic(dev) -> None:
    doc = W.doc_ids_from_lengths([[300, 212]], 512).to(dev)
    q, k, v, do = _inputs(1, 8, 2, 512, 128, dev, seed=11)
    a = _run(q, k, v, do, doc)
    b = _run(q, k, v, do, doc)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


@pytest.mark.parametrize("pack", [1, 0])
def test_attention_cfg3_pack(pack, dev) -> None:
    """cfg3 shape (S=8192, Hq=32, Hkv=8, D=128): all 8 packs run, one pack x one
    KV group (4 query heads) is checked against the oracle in full (fp32 oracle
    arithmetic for speed; its formulas are pinned in float64 on the CPU)."""
    packs = W.cfg3_packs()
    S, Hq, Hkv, D = 8192, 32, 8, 128
    doc = W.doc_ids_from_lengths(packs, S).to(dev)
    q, k, v, do = _inputs(8, Hq, Hkv, S, D, dev, seed=3)
    out, dq, dk, dv = _run(q, k, v, do, doc)
    g = 5  # KV head 5 -> query heads 20..23
    hs = slice(4 * g, 4 * g + 4)
    sl = slice(pack, pack + 1)
    ref = OA.attention(q[sl, hs], k[sl, g : g + 1], v[sl, g : g + 1], doc[sl].cpu(),
                       do[sl, hs], dtype=torch.float32)
    _close(out[sl, hs], ref["out"], "out")
    _close(dq[sl, hs], ref["dq"], "dq")
    _close(dk[sl, g : g + 1], ref["dk"], "dk")
    _close(dv[sl, g : g + 1], ref["dv"], "dv")
    assert torch.isfinite(out.float()).all() and torch.isfinite(dq.float()).all()


def test_attention_cfg3_sampled_rows_all_packs(dev) -> None:
    """cfg3 shape, every pack and every query head (all 8 KV groups): out and dQ
    at 24 sampled query rows per pack -- each document's first and last row,
    the pack's last row and random ones -- against the float64 row oracle."""
    packs = W.cfg3_packs()
    S, Hq, Hkv, D = 8192, 32, 8, 128
    doc = W.doc_ids_from_lengths(packs, S).to(dev)
    q, k, v, do = _inputs(8, Hq, Hkv, S, D, dev, seed=4)
    out, dq, _, _ = _run(q, k, v, do, doc)
    g = torch.Generator().manual_seed(12)
    rows = []
    for lens in packs:
        starts = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)[:-1]))
        ends = torch.tensor(lens).cumsum(0) - 1
        pick = torch.cat([starts[:4], ends[:4], torch.tensor([S - 1]),
                          torch.randint(0, S, (15,), generator=g)])
        rows.append(pick.unique())
    ref = OA.attention_rows(q, k, v, doc.cpu(), do, rows)
    for b in range(8):
        _close(out[b][:, rows[b]], ref["out"][b], f"pack {b} out")
        _close(dq[b][:, rows[b]], ref["dq"][b], f"pack {b} dq")


@pytest.mark.parametrize("layout", ["mixed", "noncontiguous"])
def test_attention_large_grid_layouts(layout, dev) -> None:
    """A large-grid D 128 shape (>= 2048 query tiles per launch, no KV split) with
    long and single-token documents and a padded tail, or document ids that
    recur in several runs; every head of one KV group is checked in full
    against the oracle."""
    S, Hq, Hkv, D = 8192, 32, 8, 128
    if layout == "mixed":
        doc = W.doc_ids_from_lengths([[3000, 1, 1, 700, 64, 1990, 33, 2000]], S)  # 403 pad
    else:
        doc = torch.tensor([[(i // 300) % 5 for i in range(S)]])
    doc = doc.to(dev)
    q, k, v, do = _inputs(1, Hq, Hkv, S, D, dev, seed=21)
    out, dq, dk, dv = _run(q, k, v, do, doc)
    g = 3
    hs = slice(4 * g, 4 * g + 4)
    ref = OA.attention(q[:, hs], k[:, g : g + 1], v[:, g : g + 1], doc.cpu(), do[:, hs],
                       dtype=torch.float32)
    _close(out[:, hs], ref["out"], "out")
    _close(dq[:, hs], ref["dq"], "dq")
    _close(dk[:, g : g + 1], ref["dk"], "dk")
    _close(dv[:, g : g + 1], ref["dv"], "dv")
    assert torch.isfinite(out.float()).all()


def test_attention_kept_ds_two_quads_per_kv_head(dev) -> None:
    """Kept-dS backward with G = 8 (each KV head's dS blocks hold two quads of
    query heads, and two dQ workgroups read them), lognormal packs and a
    padded tail: every query head of KV head 1, pack 2, against the oracle."""
    B, Hq, Hkv, S, D = 8, 16, 2, 4096, 128
    rng = np.random.default_rng(5)
    lens = [W.fill_sequential(rng, S, np.log(512), 1.0, 16, S) for _ in range(B)]
    lens[2] = lens[2][:-1]  # padded tail
    doc = W.doc_ids_from_lengths(lens, S).to(dev)
    q, k, v, do = _inputs(B, Hq, Hkv, S, D, dev, seed=8)
    out, dq, dk, dv = _run(q, k, v, do, doc)
    sl, g = slice(2, 3), 1
    hs = slice(8 * g, 8 * g + 8)
    ref = OA.attention(q[sl, hs], k[sl, g : g + 1], v[sl, g : g + 1], doc[sl].cpu(), do[sl, hs],
                       dtype=torch.float32)
    _close(out[sl, hs], ref["out"], "out")
    _close(dq[sl, hs], ref["dq"], "dq")
    _close(dk[sl, g : g + 1], ref["dk"], "dk")
    _close(dv[sl, g : g + 1], ref["dv"], "dv")
    assert torch.isfinite(dq.float()).all()


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("profile", ["rising", "falling"])
def test_attention_running_max_moves(profile, D, dev) -> None:
    """Scores that rise along the sequence (the forward's running max moves
    every few sub-tiles, by up to ~40 log2 units, taking the rescaling slow
    path) or fall (the first valid sub-tile holds the max, every later one
    takes the fast path), with documents that leave some lanes' first
    sub-tiles fully masked, on the pipelined kernels (S % 64 == 0)."""
    B, Hq, Hkv, S = 1, 4, 2, 1024
    g = torch.Generator().manual_seed(31 + D)
    pos = torch.arange(S, dtype=torch.float32) / S
    ramp = 6.0 * (pos if profile == "rising" else 1.0 - pos)
    q = 0.5 + 0.1 * torch.randn(B, S, Hq, D, generator=g)
    k = ramp[None, :, None, None] + 0.3 * torch.randn(B, S, Hkv, D, generator=g)
    v = torch.randn(B, S, Hkv, D, generator=g)
    do = torch.randn(B, S, Hq, D, generator=g)
    q, k, v, do = (t.to(dev, torch.bfloat16).transpose(1, 2) for t in (q, k, v, do))
    doc = W.doc_ids_from_lengths([[40, 300, 1, 400]], S).to(dev)  # 283 pad tokens
    out, dq, dk, dv = _run(q, k, v, do, doc)
    ref = OA.attention(q, k, v, doc.cpu(), do)
    what = f"{profile} scores, D {D}"
    _close(out, ref["out"], f"{what} out")
    _close(dk, ref["dk"], f"{what} dk")
    _close(dv, ref["dv"], f"{what} dv")
    # The north star's 2e-2 bar for dQ, against the oracle whose delta is
    # formed from the stored bf16 output (as the reference's own backward
    # forms it), so the bf16 rounding of O is on both sides.
    stored = OA.attention(q, k, v, doc.cpu(), do, delta_out=out.detach().cpu())
    _close(dq, stored["dq"], f"{what} dq (delta from the stored output)")
    # dQ = scale dS K grows with |K| (entries up to ~6 here, against ~1 in the
    # N(0, 1) cases), and so does its error, which the bf16 rounding of O in
    # rowsum(dO * O) dominates (present in any bf16-output implementation):
    # the absolute tolerance is scaled by the mean |K| entry (~3).
    torch.testing.assert_close(dq.detach().float().cpu(), ref["dq"].float(), atol=3 * TOL,
                               rtol=TOL, msg=lambda m: f"{what} dq: {m}")


def _bwd_abi(q, k, v, out, do, lse, doc, outs=None):
    """pb_attn_bwd through the C ABI on given forward results; dq / dk / dv as
    [B, S, H, D] memory seen as [B, H, S, D] (the model's layout)."""
    from packbalance_amd import _native as N
    from packbalance_amd.model import attention as A

    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    plans = A._plans(doc, Hq, Hkv, D, None)
    if outs is None:
        outs = (torch.empty(B, S, Hq, D, device=q.device, dtype=q.dtype).transpose(1, 2),
                torch.empty(B, S, Hkv, D, device=q.device, dtype=q.dtype).transpose(1, 2),
                torch.empty(B, S, Hkv, D, device=q.device, dtype=q.dtype).transpose(1, 2),
                torch.empty(max(1, plans["workspace"]), dtype=torch.uint8, device=q.device))
    dq, dk, dv, ws = outs
    pq, pk = plans[A.BWD_Q], plans[A.BWD_KV]
    N.call("pb_attn_bwd", N.BHSD.of(q), N.BHSD.of(k), N.BHSD.of(v), N.BHSD.of(out),
           N.BHSD.of(do), N.BHSD.of(dq), N.BHSD.of(dk), N.BHSD.of(dv), lse.data_ptr(),
           ws.data_ptr(), doc.data_ptr(), doc.stride(0), pq.counts.data_ptr(),
           pq.lists.data_ptr(), pk.counts.data_ptr(), pk.lists.data_ptr(), B, Hq, Hkv, S, D,
           1.0 / math.sqrt(D), N.PB_BF16, N.stream_ptr(q))
    return outs


def _fwd_abi(q, k, v, doc):
    from packbalance_amd import _native as N
    from packbalance_amd.model import attention as A

    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    plans = A._plans(doc, Hq, Hkv, D, None)
    out = torch.empty(B, S, Hq, D, device=q.device, dtype=q.dtype).transpose(1, 2)
    lse = torch.empty(B, Hq, S, device=q.device, dtype=torch.float32)
    fws = torch.empty(max(1, plans["fwd_workspace"]), dtype=torch.uint8, device=q.device)
    p = plans[A.FWD]
    N.call("pb_attn_fwd", N.BHSD.of(q), N.BHSD.of(k), N.BHSD.of(v), N.BHSD.of(out),
           lse.data_ptr(), fws.data_ptr(), doc.data_ptr(), doc.stride(0), p.counts.data_ptr(),
           p.lists.data_ptr(), B, Hq, Hkv, S, D, 1.0 / math.sqrt(D), N.PB_BF16,
           N.stream_ptr(q))
    return out, lse


def test_kept_ds_backward_packs_independent(dev) -> None:
    """The kept-dS backward (dK/dV storing dS, then dQ from it) is independent
    of the batch around a pack: the gradients of a 4-pack call equal, bit for
    bit, those of each pack alone, on the same forward results (per-pack
    offsets of the plans, the dS blocks, lse and delta)."""
    B, Hq, Hkv, S, D = 4, 32, 8, 8192, 128
    doc = W.doc_ids_from_lengths(W.cfg3_packs()[:B], S).to(dev)
    q, k, v, do = _inputs(B, Hq, Hkv, S, D, dev, seed=21)
    out, lse = _fwd_abi(q, k, v, doc)
    dq, dk, dv, _ = _bwd_abi(q, k, v, out, do, lse, doc)
    for b in range(B):
        sl = slice(b, b + 1)
        dq1, dk1, dv1, _ = _bwd_abi(q[sl], k[sl], v[sl], out[sl], do[sl], lse[sl],
                                    doc[sl].contiguous())
        for name, got, want in (("dq", dq[sl], dq1), ("dk", dk[sl], dk1), ("dv", dv[sl], dv1)):
            assert torch.equal(got, want), f"pack {b} {name} differs from the single-pack call"
    assert torch.isfinite(dq.float()).all() and torch.isfinite(dk.float()).all()


def test_kept_ds_backward_graph_replays(dev) -> None:
    """The kept-dS backward captured into a HIP graph: every replay, with eager
    work and synchronisations between them and the outputs poisoned before
    each, gives the eager call's gradients bit for bit."""
    B, Hq, Hkv, S, D = 2, 32, 8, 8192, 128
    doc = W.doc_ids_from_lengths(W.cfg3_packs()[1 : 1 + B], S).to(dev)
    q, k, v, do = _inputs(B, Hq, Hkv, S, D, dev, seed=22)
    out, lse = _fwd_abi(q, k, v, doc)
    want = [t.clone() for t in _bwd_abi(q, k, v, out, do, lse, doc)[:3]]
    torch.cuda.synchronize()
    outs = _bwd_abi(q, k, v, out, do, lse, doc)  # static outputs and workspace
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _bwd_abi(q, k, v, out, do, lse, doc, outs)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _bwd_abi(q, k, v, out, do, lse, doc, outs)
    for rep in range(3):
        for t in outs[:3]:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, got, w in zip(("dq", "dk", "dv"), outs[:3], want):
            assert torch.equal(got, w), f"replay {rep}: {name} differs from the eager call"
        _ = (q.float() * 2).sum().item()  # eager work between replays
