"""GPU parity: RMSNorm and SwiGLU kernels vs the CPU oracle.

Tolerances (torch.testing semantics, |a-b| <= atol + rtol*|b|):
  fp32 activations: 1e-5;  bf16 activations: 1e-2 (the hot-path bar for
  RMSNorm and SwiGLU).  The reference's own GPU test uses 2e-2
  (tests/test_kernels.py:107-142).
"""

from __future__ import annotations

import pytest
import torch

from oracle import kernels as OK
from packbalance_amd import _native as N
from packbalance_amd.kernels.rmsnorm import rmsnorm
from packbalance_amd.kernels.swiglu import swiglu

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2, torch.float16: 1e-2}


def _close(got: torch.Tensor, want: torch.Tensor, tol: float, what: str) -> None:
    torch.testing.assert_close(got.detach().cpu().double(), want.double(), rtol=tol, atol=tol,
                               msg=lambda m: f"{what}: {m}")


def _rms_case(shape, dtype, wdtype, dev, *, seed=0, row_view=False, wstd=1.0, wmean=0.0):
    g = torch.Generator().manual_seed(seed)
    n = shape[-1]
    if row_view:
        base = torch.randn(*shape[:-1], n + 24, generator=g)
        x = base.to(dev, dtype)[..., 5 : 5 + n]
    else:
        x = torch.randn(*shape, generator=g).to(dev, dtype)
    w = (torch.randn(n, generator=g) * wstd + wmean).to(dev, wdtype)
    dy = torch.randn(*shape, generator=g).to(dev, dtype)
    return x, w, dy


@pytest.mark.parametrize(
    "shape,dtype,wdtype",
    [
        ((32, 64), torch.float32, torch.float32),  # reference GPU test shape
        ((8, 32), torch.float32, torch.float32),
        ((2048, 768), torch.float32, torch.float32),  # model dtype flow (fp32 residual)
        ((4, 7, 768), torch.bfloat16, torch.float32),
        ((513, 4096), torch.bfloat16, torch.bfloat16),
        ((64, 100), torch.float32, torch.float32),  # n not a multiple of the vector
        ((33, 8192), torch.bfloat16, torch.bfloat16),  # streaming (non-register) rows
        ((16, 96), torch.float16, torch.float32),
        ((37, 1024), torch.float32, torch.float32),  # column-split backward, 1 vector per lane
        ((130, 2048), torch.bfloat16, torch.float32),  # column-split, ragged last batch
        ((9, 4096), torch.float16, torch.float16),  # column-split, 2 vectors per lane
        # several rows per backward wave (more rows than the grid's waves), the last
        # pass ragged: the next row's loads issue as the current row's dx leaves
        ((4100, 1024), torch.bfloat16, torch.bfloat16),
        ((4100, 1000), torch.bfloat16, torch.float32),  # inactive lanes in the last vector
        ((5000, 768), torch.float32, torch.float32),
    ],
)
def test_rmsnorm_matches_oracle(shape, dtype, wdtype, dev) -> None:
    eps = 1e-5
    x, w, dy = _rms_case(shape, dtype, wdtype, dev)
    xr = x.clone().requires_grad_(True)
    wr = w.clone().requires_grad_(True)
    y = rmsnorm(xr, wr, eps)
    y.backward(dy)
    tol = TOL[dtype]
    y_ref, _ = OK.rmsnorm_fwd(x, w, eps)
    dx_ref, dw_ref = OK.rmsnorm_bwd(dy, x, w, eps)
    assert y.dtype == dtype and y.shape == x.shape
    assert xr.grad.dtype == dtype and wr.grad.dtype == wdtype
    _close(y, y_ref, tol, "y")
    _close(xr.grad, dx_ref, tol, "dx")
    # dw sums over all rows; compare relative to its scale.
    _close(wr.grad, dw_ref, max(tol, 1e-4), "dw")


def test_rmsnorm_strided_rows(dev) -> None:
    # Rows of a wider buffer (row stride 280, base offset 20 bytes).
    x, w, dy = _rms_case((64, 256), torch.float32, torch.float32, dev, row_view=True)
    assert not x.is_contiguous()
    xr = x.detach().requires_grad_(True)
    y = rmsnorm(xr, w, 1e-5)
    y.backward(dy)
    _close(y, OK.rmsnorm_fwd(x, w, 1e-5)[0], 1e-5, "y (strided)")
    _close(xr.grad, OK.rmsnorm_bwd(dy, x, w, 1e-5)[0], 1e-5, "dx (strided)")


def test_rmsnorm_cfg5_full_size(dev) -> None:
    """cfg5: x [32768, 4096] bf16 ~N(0,1), w ~N(1, 0.1), eps 1e-5, dy ~N(0,1).

    y and dx are row-local: checked on 512 sampled rows against the fp64
    oracle; dw (a sum over every row) is checked in full.
    """
    eps = 1e-5
    x, w, dy = _rms_case((32768, 4096), torch.bfloat16, torch.bfloat16, dev, wstd=0.1, wmean=1.0)
    xr = x.clone().requires_grad_(True)
    wr = w.clone().requires_grad_(True)
    y = rmsnorm(xr, wr, eps)
    y.backward(dy)
    rows = torch.randperm(32768, generator=torch.Generator().manual_seed(5))[:512]
    rd = rows.to(dev)
    _close(y[rd], OK.rmsnorm_fwd(x[rd], w, eps)[0], 1e-2, "y")
    _close(xr.grad[rd], OK.rmsnorm_bwd(dy[rd], x[rd], w, eps)[0], 1e-2, "dx")
    _, dw_ref = OK.rmsnorm_bwd(dy, x, w, eps)
    _close(wr.grad, dw_ref, 1e-2, "dw")


def _bwd_abi(dy, x, w, rstd, ws):
    rows, n = x.shape
    dx, dw = torch.empty_like(x), torch.empty_like(w)
    N.call("pb_rmsnorm_bwd", dy.data_ptr(), dy.stride(0), x.data_ptr(), x.stride(0),
           N.dtype_code(x), w.data_ptr(), N.dtype_code(w), rstd.data_ptr(), dx.data_ptr(),
           dx.stride(0), dw.data_ptr(), ws.data_ptr(), rows, n, N.stream_ptr(x))
    return dx, dw


@pytest.mark.parametrize("rows,n,dtype", [
    (32768, 4096, torch.bfloat16),  # 512 workgroups: 512 dW partial rows
    (40, 768, torch.float32),       # 5 workgroups
    (8, 4096, torch.bfloat16),      # one workgroup, one partial row
    (3000, 99, torch.float32),      # n % 4 != 0: the streaming kernel
])
def test_rmsnorm_bwd_workspace_reuse(rows, n, dtype, dev) -> None:
    """One workspace serves call after call (sizes changing, stale partial rows of a
    larger call left in it): results repeat bit for bit and dw matches the oracle."""
    x, w, dy = _rms_case((rows, n), dtype, dtype, dev, seed=3)
    rstd = torch.rsqrt(x.float().pow(2).mean(-1) + 1e-5).contiguous()
    ws = torch.empty(N.lib().pb_rmsnorm_bwd_workspace_bytes(32768, 4096) + 4096,
                     dtype=torch.uint8, device=dev)
    assert N.lib().pb_rmsnorm_bwd_workspace_bytes(rows, n) <= ws.numel()
    ws.fill_(0x7f)  # stale contents: every partial row must be written before it is read
    first = _bwd_abi(dy, x, w, rstd, ws)
    for _ in range(2):
        dx, dw = _bwd_abi(dy, x, w, rstd, ws)
        torch.cuda.synchronize()
        assert torch.equal(dx, first[0]) and torch.equal(dw, first[1])
    _, dw_ref = OK.rmsnorm_bwd(dy, x, w, 1e-5)
    _close(first[1], dw_ref, max(TOL[dtype], 1e-4), "dw")


def test_rmsnorm_bwd_graph_replays(dev) -> None:
    """The backward (fused dx + dW partials, then the dW reduce) captured in a HIP graph:
    every replay, with eager work between them, equals the eager result."""
    x, w, dy = _rms_case((4096, 4096), torch.bfloat16, torch.bfloat16, dev, seed=4)
    xr = x.clone().requires_grad_(True)
    wr = w.clone().requires_grad_(True)
    rmsnorm(xr, wr, 1e-5).backward(dy)  # eager
    want_dx, want_dw = xr.grad.clone(), wr.grad.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            xr.grad = wr.grad = None
            rmsnorm(xr, wr, 1e-5).backward(dy)
    torch.cuda.current_stream().wait_stream(s)
    xr.grad = wr.grad = None
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        y = rmsnorm(xr, wr, 1e-5)
        y.backward(dy)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(xr.grad, want_dx) and torch.equal(wr.grad, want_dw)
        rmsnorm(xr.detach(), w, 1e-5).sum().item()  # eager work between replays


def test_rmsnorm_rejects_cpu_and_huge() -> None:
    with pytest.raises(RuntimeError):
        rmsnorm(torch.randn(2, 8), torch.ones(8), 1e-5)
    with pytest.raises(RuntimeError):
        rmsnorm(torch.randn(1, 70000, device="cuda"), torch.ones(70000, device="cuda"), 1e-5)


@pytest.mark.parametrize(
    "shape,dtype",
    [
        ((16, 32), torch.float32),  # reference GPU test shape
        ((8, 16), torch.float32),
        ((1, 2048, 2048), torch.bfloat16),  # model call site
        ((7, 333), torch.bfloat16),  # scalar tail
        ((5, 64), torch.float16),
    ],
)
def test_swiglu_matches_oracle(shape, dtype, dev) -> None:
    g0 = torch.Generator().manual_seed(0)
    gate = torch.randn(*shape, generator=g0).to(dev, dtype)
    up = torch.randn(*shape, generator=g0).to(dev, dtype)
    dy = torch.randn(*shape, generator=g0).to(dev, dtype)
    gr = gate.clone().requires_grad_(True)
    ur = up.clone().requires_grad_(True)
    out = swiglu(gr, ur)
    out.backward(dy)
    tol = TOL[dtype]
    _close(out, OK.swiglu_fwd(gate, up), tol, "out")
    dg, du = OK.swiglu_bwd(gate, up, dy)
    _close(gr.grad, dg, tol, "dgate")
    _close(ur.grad, du, tol, "dup")


def test_swiglu_cfg5_full_size(dev) -> None:
    """cfg5: gate/up [32768, 14336] bf16 ~N(0,1), dy ~N(0,1).

    1M sampled elements against the fp64 oracle, every element against a
    torch fp32 evaluation of the same formula on the device.
    """
    torch.manual_seed(0)
    shape = (32768, 14336)
    gate = torch.randn(shape, device=dev, dtype=torch.bfloat16)
    up = torch.randn(shape, device=dev, dtype=torch.bfloat16)
    dy = torch.randn(shape, device=dev, dtype=torch.bfloat16)
    gr = gate.clone().requires_grad_(True)
    ur = up.clone().requires_grad_(True)
    out = swiglu(gr, ur)
    out.backward(dy)
    idx = torch.randint(0, gate.numel(), (1 << 20,), device=dev)
    gf, uf, df = (t.reshape(-1)[idx] for t in (gate, up, dy))
    _close(out.reshape(-1)[idx], OK.swiglu_fwd(gf, uf), 1e-2, "out (sampled)")
    dg, du = OK.swiglu_bwd(gf, uf, df)
    _close(gr.grad.reshape(-1)[idx], dg, 1e-2, "dgate (sampled)")
    _close(ur.grad.reshape(-1)[idx], du, 1e-2, "dup (sampled)")
    # Whole tensors against torch fp32, chunked to bound memory.
    for r in range(0, shape[0], 4096):
        g, u, d = (t[r : r + 4096].float() for t in (gate, up, dy))
        s = torch.sigmoid(g)
        torch.testing.assert_close(out[r : r + 4096].float(), g * s * u, rtol=1e-2, atol=1e-2)
        torch.testing.assert_close(gr.grad[r : r + 4096].float(), d * u * s * (1 + g * (1 - s)),
                                   rtol=1e-2, atol=1e-2)
        torch.testing.assert_close(ur.grad[r : r + 4096].float(), d * g * s, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize(
    "rows,cols,dtype",
    [
        (2048, 2048, torch.bfloat16),  # cfg2 fused gate|up projection
        (256, 344, torch.bfloat16),  # cfg1 ffn
        (37, 333, torch.bfloat16),  # cols % 8 != 0: scalar path
        (64, 96, torch.float32),
    ],
)
def test_swiglu_rows_on_fused_halves_match_oracle(rows, cols, dtype, dev) -> None:
    """gate/up are the halves of one [rows, 2*cols] buffer and dgate/dup are written
    back into one such buffer (pb_swiglu_fwd_rows / pb_swiglu_bwd_rows)."""
    g0 = torch.Generator().manual_seed(1)
    gu = torch.randn(rows, 2 * cols, generator=g0).to(dev, dtype)
    dy = torch.randn(rows, cols, generator=g0).to(dev, dtype)
    gate, up = gu[:, :cols], gu[:, cols:]
    out = torch.full((rows, cols), float("nan"), dtype=dtype, device=dev)
    st, code = N.stream_ptr(gu), N.dtype_code(gu)
    N.call("pb_swiglu_fwd_rows", gate.data_ptr(), 2 * cols, up.data_ptr(), 2 * cols,
           out.data_ptr(), cols, rows, cols, code, st)
    dgu = torch.full_like(gu, float("nan"))
    N.call("pb_swiglu_bwd_rows", gate.data_ptr(), 2 * cols, up.data_ptr(), 2 * cols,
           dy.data_ptr(), cols, dgu.data_ptr(), 2 * cols, dgu[:, cols:].data_ptr(), 2 * cols,
           rows, cols, code, st)
    tol = TOL[dtype]
    _close(out, OK.swiglu_fwd(gate, up), tol, "out")
    dg, du = OK.swiglu_bwd(gate, up, dy)
    _close(dgu[:, :cols], dg, tol, "dgate")
    _close(dgu[:, cols:], du, tol, "dup")


def test_swiglu_rows_rejects_bad_strides(dev) -> None:
    x = torch.zeros(4, 8, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        N.call("pb_swiglu_fwd_rows", x.data_ptr(), 4, x.data_ptr(), 8, x.data_ptr(), 8, 4, 8,
               N.dtype_code(x), N.stream_ptr(x))


def test_swiglu_rejects_cpu() -> None:
    with pytest.raises(RuntimeError):
        swiglu(torch.randn(4), torch.randn(4))


# ---------------------------------------------------------------- fused residual add + RMSNorm
@pytest.mark.parametrize(
    "rows,n,xdt,ddt,ydt,wdt",
    [
        (2048, 768, torch.float32, torch.bfloat16, torch.bfloat16, torch.float32),  # cfg2 flow
        (300, 2048, torch.float32, torch.bfloat16, torch.bfloat16, torch.float32),  # 4 vectors/lane
        (64, 512, torch.bfloat16, torch.bfloat16, torch.bfloat16, torch.bfloat16),
        (40, 4096, torch.float32, torch.float32, torch.bfloat16, torch.float32),  # loop kernel
        (37, 100, torch.float32, torch.float16, torch.float32, torch.float32),  # n % 8 != 0
    ],
)
def test_add_rmsnorm_matches_oracle(rows, n, xdt, ddt, ydt, wdt, dev) -> None:
    from packbalance_amd.kernels.rmsnorm import add_rmsnorm

    g = torch.Generator().manual_seed(rows + n)
    x = torch.randn(rows, n, generator=g).to(dev, xdt)
    d = torch.randn(rows, n, generator=g).to(dev, ddt)
    w = (torch.randn(n, generator=g) * 0.1 + 1.0).to(dev, wdt)
    dy = torch.randn(rows, n, generator=g).to(dev, ydt)
    dres = torch.randn(rows, n, generator=g).to(dev, xdt)
    xr, dr, wr = (t.clone().requires_grad_(True) for t in (x, d, w))
    h, y = add_rmsnorm(xr, dr, wr, 1e-5, out_dtype=ydt)
    assert h.dtype == xdt and y.dtype == ydt
    torch.autograd.backward((h, y), (dres, dy))
    h_ref, y_ref, _ = OK.add_rmsnorm_fwd(x, d, w, 1e-5)
    gx_ref, gw_ref = OK.add_rmsnorm_bwd(dy, dres, h_ref, w, 1e-5)
    _close(h, h_ref, TOL[xdt], "h")
    _close(y, y_ref, TOL[ydt], "y")
    _close(xr.grad, gx_ref, TOL[xdt] if xdt == torch.float32 else 2e-2, "dx")
    _close(dr.grad, gx_ref, TOL[ddt], "ddelta")
    assert xr.grad.dtype == xdt and dr.grad.dtype == ddt and wr.grad.dtype == wdt
    _close(wr.grad, gw_ref, max(TOL[ydt], 1e-4) * 10, "dw")


def test_rmsnorm_to_bf16_matches_oracle(dev) -> None:
    """fp32 residual in, bf16 activations out (the model's first norm); dx back in fp32."""
    from packbalance_amd.kernels.rmsnorm import rmsnorm_to

    x, w, _ = _rms_case((512, 768), torch.float32, torch.float32, dev, seed=3)
    dy = torch.randn(512, 768, device=dev).to(torch.bfloat16)
    xr, wr = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    y = rmsnorm_to(xr, wr, 1e-5, torch.bfloat16)
    assert y.dtype == torch.bfloat16
    y.backward(dy)
    y_ref, _ = OK.rmsnorm_fwd(x, w, 1e-5)
    dx_ref, dw_ref = OK.rmsnorm_bwd(dy, x, w, 1e-5)
    _close(y, y_ref, 1e-2, "y")
    _close(xr.grad, dx_ref, 1e-5, "dx")
    _close(wr.grad, dw_ref, 1e-4, "dw")


@pytest.mark.parametrize("rows,n", [(2048, 768), (40, 4096), (0, 768)])
def test_norm_weight_grad_accumulates_into_fp32_buffer(rows, n, dev) -> None:
    """dw_acc: the weight gradient is ADDED to a caller's fp32 buffer (the flat
    store's slice) and None is returned for the weight; the increase equals the dw
    the non-accumulating call returns (same kernel, same reduction order), and an
    empty batch leaves the buffer unchanged."""
    from packbalance_amd.kernels.rmsnorm import add_rmsnorm, rmsnorm_to

    g = torch.Generator().manual_seed(7)
    x = torch.randn(rows, n, generator=g).to(dev)
    d = torch.randn(rows, n, generator=g).to(dev, torch.bfloat16)
    w = (torch.randn(n, generator=g) * 0.1 + 1.0).to(dev)
    dy = torch.randn(rows, n, generator=g).to(dev, torch.bfloat16)
    acc0 = torch.randn(n, generator=g).to(dev)
    for fused in (True, False):
        wr = w.clone().requires_grad_(True)
        wa = w.clone().requires_grad_(True)
        acc = acc0.clone()
        if fused:
            _, y = add_rmsnorm(x, d, wr, 1e-5, torch.bfloat16)
            _, ya = add_rmsnorm(x, d, wa, 1e-5, torch.bfloat16, dw_acc=acc)
        else:
            y = rmsnorm_to(x, wr, 1e-5, torch.bfloat16)
            ya = rmsnorm_to(x, wa, 1e-5, torch.bfloat16, dw_acc=acc)
        if rows == 0:
            assert wa.grad is None
            continue
        y.backward(dy)
        ya.backward(dy)
        assert wa.grad is None
        torch.testing.assert_close(acc - acc0, wr.grad, rtol=1e-5, atol=1e-4)
    with pytest.raises(ValueError):
        add_rmsnorm(x, d, w.to(torch.bfloat16), 1e-5, dw_acc=acc0)


def test_norm_weight_grad_deferred_to_a_batched_reduce(dev) -> None:
    """dw_defer: 35 norms of one backward pass (slot 0 an rmsnorm_to, the rest
    add_rmsnorm; slot 5 unused) leave their dw partials in a WgradPlan, which adds
    them to their fp32 buffers when the pass ends, in two runs of consecutive
    slots (the second, 30 norms, plus the first's 5, launched as 32-problem
    batches); every buffer and dx equal the immediate dw_acc path bit for bit."""
    from packbalance_amd.kernels.rmsnorm import add_rmsnorm, rmsnorm_to
    from packbalance_amd.model.layers import WgradPlan

    rows, n, count = 4096, 768, 36
    g = torch.Generator().manual_seed(11)
    xs = [torch.randn(rows, n, generator=g).to(dev) for _ in range(count)]
    ds = [torch.randn(rows, n, generator=g).to(dev, torch.bfloat16) for _ in range(count)]
    ws = [(torch.randn(n, generator=g) * 0.1 + 1.0).to(dev) for _ in range(count)]
    dys = [torch.randn(rows, n, generator=g).to(dev, torch.bfloat16) for _ in range(count)]
    acc0 = torch.randn(count, n, generator=g).to(dev)
    slots = [i for i in range(count) if i != 5]
    plan = WgradPlan(1, rows, {}, torch.bfloat16, dev, norms=count, norm_dim=n)

    def run(defer):
        acc = acc0.clone()
        xr = [x.clone().requires_grad_(True) for x in xs]
        outs = []
        for i in slots:
            kw = dict(dw_acc=acc[i], dw_defer=(plan, i) if defer else None)
            if i == 0:
                outs.append(rmsnorm_to(xr[i], ws[i], 1e-5, torch.bfloat16, **kw))
            else:
                outs.append(add_rmsnorm(xr[i], ds[i], ws[i], 1e-5, torch.bfloat16, **kw)[1])
        torch.autograd.backward(outs, [dys[i] for i in slots])
        return acc, [xr[i].grad for i in slots]

    before = WgradPlan.norm_reduces
    acc_d, dx_d = run(True)
    assert WgradPlan.norm_reduces - before == 2
    acc_i, dx_i = run(False)
    assert torch.equal(acc_d, acc_i)
    assert torch.equal(acc_d[5], acc0[5])
    assert all(torch.equal(a, b) for a, b in zip(dx_d, dx_i))
    assert not torch.equal(acc_d, acc0)
