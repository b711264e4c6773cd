"""GPU parity: fused LM-head cross-entropy (loss, dx, dW) vs the oracle.

The oracle is float64 CE over the bf16-rounded x and W (the kernel's operands;
the reference's autocast GEMM rounds them the same way); fp32 x and W outside
autocast take the fp32 path (an fp32 product, as the reference's) and are
checked against the oracle on the fp32 inputs at fp32-level tolerances.  Tolerances: loss
within 1e-4 relative (the CE bar); dx / dW (computed from bf16 dlogits)
within 2e-2 (the reference GPU test's tolerance, tests/test_kernels.py:84-104)
and within 1e-2 in relative Frobenius norm.  Both backward paths are run:
recomputing the logits (the default: logits budget 0, no full logits) and from
the logits the forward kept (a budget that holds them).
"""

from __future__ import annotations

import pytest
import torch

from oracle import kernels as OK
from packbalance_amd.kernels import fused_ce as FC
from packbalance_amd.kernels.fused_ce import linear_cross_entropy

pytestmark = pytest.mark.gpu
KEEP = 16 << 30  # a logits budget that holds every case's logits (cfg4: 4.2 GB)


def _rel_fro(got: torch.Tensor, want: torch.Tensor) -> float:
    g, w = got.detach().double().cpu(), want.double().cpu()
    return float((g - w).norm() / w.norm().clamp_min(1e-30))


def _case(n_shape, v, d, xdtype, wdtype, dev, *, seed=0, wstd=1.0, ignore_every=0, ignore_p=0.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*n_shape, d, generator=g).to(dev, xdtype)
    w = (torch.randn(v, d, generator=g) * wstd).to(dev, wdtype)
    t = torch.randint(0, v, n_shape, generator=g)
    if ignore_every:
        t.view(-1)[::ignore_every] = -100
    if ignore_p:
        t[torch.rand(n_shape, generator=g) < ignore_p] = -100
    return x, w, t.to(dev)


def _oracle_logits(x, w):
    """The oracle's logits rounding: bf16 where the kernels' logits are bf16 (the
    reference's product of bf16 operands), none for fp32 logits."""
    return torch.bfloat16 if FC.logits_dtype_for(x.dtype, w.dtype) == torch.bfloat16 else None


def _check(x, w, t, z, what, *, chunk=1024):
    xr = x.detach().requires_grad_(True)
    wr = w.detach().requires_grad_(True)
    loss = linear_cross_entropy(xr, wr, t, chunk_size=chunk, z_loss_coeff=z)
    loss.backward()
    if FC._fp32_operands(x, w):
        # fp32 operands: an fp32 product, as the reference's; fp32-level tolerances
        l_ref, dx_ref, dw_ref = OK.linear_ce(x, w, t, z_loss_coeff=z)
        ltol, gtol, fro = 1e-5, 1e-4, 1e-5
    else:
        l_ref, dx_ref, dw_ref = OK.linear_ce(x.to(torch.bfloat16), w.to(torch.bfloat16), t,
                                             z_loss_coeff=z, logits_dtype=_oracle_logits(x, w))
        ltol, gtol, fro = 1e-4, 2e-2, 1e-2
    assert loss.dtype == torch.float32 and loss.dim() == 0
    torch.testing.assert_close(loss.double().cpu(), l_ref, rtol=ltol, atol=ltol,
                               msg=lambda m: f"{what} loss: {m}")
    assert xr.grad.shape == x.shape and xr.grad.dtype == x.dtype
    assert wr.grad.shape == w.shape and wr.grad.dtype == w.dtype
    torch.testing.assert_close(xr.grad.double().cpu(), dx_ref, rtol=gtol, atol=gtol,
                               msg=lambda m: f"{what} dx: {m}")
    torch.testing.assert_close(wr.grad.double().cpu(), dw_ref, rtol=gtol, atol=gtol,
                               msg=lambda m: f"{what} dw: {m}")
    assert _rel_fro(xr.grad, dx_ref) < fro, what
    assert _rel_fro(wr.grad, dw_ref) < fro, what


def test_reference_gpu_case(dev) -> None:
    """tests/test_kernels.py:84-104: x [2,32,32] fp32, w [128,32], every 5th ignored, z=0.01."""
    torch.manual_seed(0)
    x = torch.randn(2, 32, 32, device=dev)
    w = torch.randn(128, 32, device=dev)
    t = torch.randint(0, 128, (2, 32), device=dev)
    t[:, ::5] = -100
    _check(x, w, t, 0.01, "reference case", chunk=16)


_CE_CASES = [
    ((37,), 64, 32, torch.float32, torch.float32, 0.0),
    ((37,), 64, 32, torch.float32, torch.float32, 0.01),
    ((300,), 1000, 96, torch.bfloat16, torch.bfloat16, 0.0),
    ((129,), 8200, 64, torch.bfloat16, torch.bfloat16, 0.0),  # 2 vocab chunks, ragged
    ((4, 50), 517, 44, torch.float32, torch.float32, 0.0),  # d % 8 != 0, v odd
    ((61,), 300, 13, torch.bfloat16, torch.bfloat16, 0.01),  # d % 8 == 5, bf16
    ((2048,), 32000, 768, torch.float32, torch.float32, 0.0),  # cfg2 dtype flow
    ((192,), 4160, 128, torch.bfloat16, torch.bfloat16, 0.01),  # DMA GEMMs, ragged tiles
    ((1030,), 66000, 64, torch.bfloat16, torch.bfloat16, 0.0),  # 256x256 lse tiles, ragged
    ((3,), 5000, 64, torch.bfloat16, torch.bfloat16, 0.01),  # DMA tiles almost all past N
]

# fp32 x and W take the fp32 path, which keeps no kernel logits: recompute only.
_CE_PARAMS = [pytest.param(*c, stored, id=f"{i}-{'stored' if stored else 'recompute'}")
              for i, c in enumerate(_CE_CASES) for stored in (True, False)
              if not (stored and c[3] == torch.float32 and c[4] == torch.float32)]


@pytest.mark.parametrize("shape,v,d,xdt,wdt,z,stored", _CE_PARAMS)
def test_fused_ce_matches_oracle(shape, v, d, xdt, wdt, z, stored, dev) -> None:
    x, w, t = _case(shape, v, d, xdt, wdt, dev, seed=v + d, wstd=0.05 if d >= 256 else 1.0,
                    ignore_every=7)
    n = x.numel() // d
    with FC.logits_budget(KEEP if stored else None):
        assert FC.stores_logits(n, v, FC.logits_dtype_for(xdt, wdt)) == stored
        _check(x, w, t, z, f"{shape}x{v}x{d}")


@pytest.mark.parametrize("lg_dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("n,v,d", [(300, 1000, 96), (129, 8200, 64), (37, 64, 32),
                                   (1030, 66000, 64), (61, 300, 16)])
def test_stored_logits_are_the_product(n, v, d, lg_dtype, dev) -> None:
    """The forward's stored logits^T [v, round8(n)]: the fp32 product of the bf16
    operands (within fp32 summation-order error), rounded to bf16 for bf16 logits
    (within one bf16 rounding of torch's fp32 product); lse and the loss of the same
    forward are those of exactly the stored values."""
    g = torch.Generator().manual_seed(n + v)
    x = torch.randn(n, d, generator=g).to(dev, torch.bfloat16)
    w = (torch.randn(v, d, generator=g) * 0.5).to(dev, torch.bfloat16)
    t = torch.randint(0, v, (n,), generator=g).to(dev)
    xb, wb = FC._bf16_rows(x), FC._bf16_rows(w)
    lse = torch.empty(n, dtype=torch.float32, device=dev)
    rows = torch.empty(n, dtype=torch.float32, device=dev)
    total = torch.zeros((), dtype=torch.float32, device=dev)
    with FC.logits_budget(KEEP):
        lg = FC._ce_forward(xb, wb, t.to(torch.int64), n, v, xb.shape[1], -100, 0.0, rows, lse,
                            total, dev, FC.N.stream_ptr(x), lg_dtype)
    assert lg is not None and lg.shape == (v, (n + 7) // 8 * 8) and lg.dtype == lg_dtype
    want = (w.float() @ x.float().t())  # [v, n] fp32
    got = lg[:, :n].float()
    err = (got - want).abs()
    if lg_dtype == torch.bfloat16:
        tol = want.abs() * torch.finfo(torch.bfloat16).eps + 1e-5
    else:
        tol = want.abs() * 1e-5 + 1e-5
    assert bool((err <= tol).all()), float((err / want.abs().clamp_min(1e-6)).max())
    # lse and per-row loss from exactly the stored values
    got64 = got.double()
    torch.testing.assert_close(lse.double(), torch.logsumexp(got64.t(), dim=-1), rtol=1e-5,
                               atol=1e-5)
    tl = got64.t().gather(1, t[:, None].long())[:, 0]
    torch.testing.assert_close(rows.double(), torch.logsumexp(got64.t(), dim=-1) - tl,
                               rtol=1e-5, atol=1e-5)


def test_fused_ce_all_ignored_and_empty(dev) -> None:
    x = torch.randn(9, 16, device=dev, requires_grad=True)
    w = torch.randn(24, 16, device=dev, requires_grad=True)
    t = torch.full((9,), -100, device=dev)
    loss = linear_cross_entropy(x, w, t)
    loss.backward()
    assert float(loss) == 0.0
    assert float(x.grad.abs().sum()) == 0.0 and float(w.grad.abs().sum()) == 0.0
    x0 = torch.randn(0, 16, device=dev, requires_grad=True)
    l0 = linear_cross_entropy(x0, w, torch.zeros(0, dtype=torch.long, device=dev))
    l0.backward()
    assert float(l0) == 0.0 and x0.grad.shape == (0, 16)


def test_fused_ce_errors(dev) -> None:
    with pytest.raises(ValueError):
        linear_cross_entropy(torch.randn(4, 8, device=dev), torch.randn(5, 8, device=dev),
                             torch.zeros(3, dtype=torch.long, device=dev))
    with pytest.raises(RuntimeError):
        linear_cross_entropy(torch.randn(4, 8), torch.randn(5, 8), torch.zeros(4, dtype=torch.long))


def test_fused_ce_grad_output_scaling(dev) -> None:
    x, w, t = _case((64,), 300, 32, torch.bfloat16, torch.bfloat16, dev, seed=5)
    xr = x.detach().requires_grad_(True)
    wr = w.detach().requires_grad_(True)
    (linear_cross_entropy(xr, wr, t) * 0.25).backward()
    _, dx_ref, dw_ref = OK.linear_ce(x, w, t, logits_dtype=_oracle_logits(x, w))
    torch.testing.assert_close(xr.grad.double().cpu(), dx_ref * 0.25, rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(wr.grad.double().cpu(), dw_ref * 0.25, rtol=2e-2, atol=2e-2)


def test_fused_ce_fp32_inputs_under_bf16_autocast(dev) -> None:
    """The model's cfg2 flow (packbalance/model/llama.py:225): fp32 hidden states and the
    fp32 tied weight under bf16 autocast.  The reference's product is then bf16 (autocast), so the kernel
    path runs with bf16 operands and bf16 logits, against that oracle."""
    x, w, t = _case((2048,), 32000, 768, torch.float32, torch.float32, dev, seed=11, wstd=0.05,
                    ignore_every=7)
    xr = x.detach().requires_grad_(True)
    wr = w.detach().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        assert not FC._fp32_operands(x, w)
        loss = linear_cross_entropy(xr, wr, t)
    loss.backward()
    l_ref, dx_ref, dw_ref = OK.linear_ce(x.to(torch.bfloat16), w.to(torch.bfloat16), t,
                                         logits_dtype=torch.bfloat16)
    torch.testing.assert_close(loss.double().cpu(), l_ref, rtol=1e-4, atol=1e-4)
    assert xr.grad.dtype == torch.float32 and wr.grad.dtype == torch.float32
    torch.testing.assert_close(xr.grad.double().cpu(), dx_ref, rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(wr.grad.double().cpu(), dw_ref, rtol=2e-2, atol=2e-2)
    assert _rel_fro(xr.grad, dx_ref) < 1e-2 and _rel_fro(wr.grad, dw_ref) < 1e-2


def test_fused_ce_fp32_path_grad_output_scaling(dev) -> None:
    """fp32 x and W (no autocast): grad_output scales dx and dW, at fp32 tolerances; a 3-D x
    keeps its shape in dx (fused_ce.py:169,194)."""
    x, w, t = _case((2, 48), 700, 40, torch.float32, torch.float32, dev, seed=9, ignore_every=5)
    assert FC._fp32_operands(x, w)
    xr = x.detach().requires_grad_(True)
    wr = w.detach().requires_grad_(True)
    (linear_cross_entropy(xr, wr, t, z_loss_coeff=0.01) * 0.25).backward()
    _, dx_ref, dw_ref = OK.linear_ce(x, w, t, z_loss_coeff=0.01)
    assert xr.grad.shape == x.shape
    torch.testing.assert_close(xr.grad.double().cpu(), dx_ref * 0.25, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(wr.grad.double().cpu(), dw_ref * 0.25, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("vchunk,stored", [(8192, True), (8192, False), (32768, True)])
def test_fused_ce_cfg4_full_size(vchunk, stored, dev) -> None:
    """cfg4: x [16384, 4096] bf16 ~N(0,1), W [128256, 4096] bf16 ~N(0, 0.02), 1% ignored,
    at the configuration's vocab chunk (8192: 15 x 8192 + 5376) and at 32768, the
    backward from the stored bf16 logits (4.2 GB) and recomputing them.

    Every output against a torch fp32 evaluation of the bf16-rounded logits (the
    bf16 product's) on the device (row chunks, never the whole [N, V] block at
    once); 32 sampled rows of loss and dx against the float64 oracle.
    """
    N, V, D = 16384, 128256, 4096
    torch.manual_seed(0)
    x = torch.randn(N, D, device=dev, dtype=torch.bfloat16)
    w = (torch.randn(V, D, device=dev) * 0.02).to(torch.bfloat16)
    t = torch.randint(0, V, (N,), device=dev)
    t[torch.rand(N, device=dev) < 0.01] = -100
    xr = x.detach().requires_grad_(True)
    wr = w.detach().requires_grad_(True)
    with FC.vocab_chunk_rows(vchunk), FC.logits_budget(KEEP if stored else None):
        assert FC.vocab_chunk(N, V) == vchunk
        assert FC.stores_logits(N, V, torch.bfloat16) == stored
        loss = linear_cross_entropy(xr, wr, t)
        loss.backward()

    wf = w.float()
    ref_loss = torch.zeros((), device=dev, dtype=torch.float64)
    dx_ref = torch.empty(N, D, device=dev)
    dw_ref = torch.zeros(V, D, device=dev)
    for r in range(0, N, 2048):
        xs = x[r : r + 2048].float()
        ts = t[r : r + 2048]
        logits = (xs @ wf.t()).to(torch.bfloat16).float()  # the bf16 product's logits
        lse = torch.logsumexp(logits, dim=-1)
        valid = ts != -100
        safe = torch.where(valid, ts, torch.zeros_like(ts))
        tl = logits.gather(1, safe[:, None])[:, 0]
        ref_loss += torch.where(valid, lse - tl, torch.zeros_like(lse)).double().sum()
        p = torch.softmax(logits, dim=-1)
        p[torch.arange(p.shape[0], device=dev), safe] -= 1.0
        p[~valid] = 0.0
        dx_ref[r : r + 2048] = p @ wf
        dw_ref += p.t() @ xs
        del logits, p
    torch.testing.assert_close(loss.double(), ref_loss, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(xr.grad.float(), dx_ref, rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(wr.grad.float(), dw_ref, rtol=2e-2, atol=2e-2)
    assert _rel_fro(xr.grad.float(), dx_ref) < 1e-2
    assert _rel_fro(wr.grad.float(), dw_ref) < 1e-2
    rows = torch.randperm(N, generator=torch.Generator().manual_seed(1))[:32].to(dev)
    l_rows, dx_rows, _ = OK.linear_ce(x[rows], w, t[rows], logits_dtype=torch.bfloat16)
    torch.testing.assert_close(dx_rows, xr.grad[rows].double().cpu(), rtol=2e-2, atol=2e-2)
    # the loss of those rows alone through the kernels, against the float64 oracle
    l_kernel = linear_cross_entropy(x[rows], w, t[rows])
    torch.testing.assert_close(l_kernel.double().cpu(), l_rows, rtol=1e-4, atol=1e-4)
