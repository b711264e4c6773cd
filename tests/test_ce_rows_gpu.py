"""GPU parity: the row cross-entropy kernel (the _ce_kernel contract) vs the oracle.

Loss and lse are compared with rtol 1e-4 (the CE bar); dlogits with the
logits dtype's resolution (fp32: 1e-5, bf16: 1e-2 absolute on values in [-1, 1]).
"""

from __future__ import annotations

import pytest
import torch

from oracle import kernels as OK
from packbalance_amd.kernels.fused_ce import ce_rows

pytestmark = pytest.mark.gpu


def _case(m, v, dtype, dev, *, seed=0, scale=1.0, ignore_every=0, transposed=False):
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(m, v, generator=g) * scale).to(dev, dtype)
    if transposed:
        logits = logits.t().contiguous().t()  # same values, stride_v = m
    t = torch.randint(0, v, (m,), generator=g)
    if ignore_every:
        t[::ignore_every] = -100
    return logits, t.to(dev)


@pytest.mark.parametrize(
    "m,v,dtype,z,transposed",
    [
        (64, 128, torch.float32, 0.0, False),
        (37, 32000, torch.float32, 0.0, False),  # model vocab, 1024-thread register rows
        (7, 40000, torch.bfloat16, 0.0, False),  # 1024-thread register rows, bf16
        (5, 33000, torch.float32, 0.0, False),  # beyond the register rows: streaming
        (16, 8192, torch.bfloat16, 0.0, False),  # register path (cfg4 chunk width)
        (16, 8192, torch.bfloat16, 0.01, False),
        (9, 1000, torch.bfloat16, 0.01, True),  # strided vocab axis
        (5, 7, torch.float32, 0.0, False),
        (3, 128256, torch.bfloat16, 0.0, False),  # full cfg4 vocab, streaming
    ],
)
def test_ce_rows_matches_oracle(m, v, dtype, z, transposed, dev) -> None:
    logits, t = _case(m, v, dtype, dev, ignore_every=5, transposed=transposed, scale=3.0)
    if transposed:
        assert logits.stride(1) != 1
    loss, lse, dl = ce_rows(logits, t, ignore_index=-100, z_loss_coeff=z, write_dlogits=True)
    l_ref, lse_ref, dl_ref = OK.ce_rows(logits, t, ignore_index=-100, z_loss_coeff=z)
    torch.testing.assert_close(loss.cpu().double(), l_ref, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(lse.cpu().double(), lse_ref, rtol=1e-4, atol=1e-4)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert dl.dtype == dtype and dl.stride() == logits.stride()
    torch.testing.assert_close(dl.cpu().double(), dl_ref, rtol=tol, atol=tol)
    ignored = (t == -100).cpu()
    assert float(loss.cpu()[ignored].abs().sum()) == 0.0
    assert float(dl.cpu()[ignored].abs().sum()) == 0.0


@pytest.mark.parametrize(
    "m,v,dtype,transposed",
    [
        (41, 32000, torch.float32, False),  # the library-GEMM CE block: fp32 in, bf16 out
        (6, 1000, torch.float32, False),  # 256-thread register rows
        (4, 33000, torch.float32, False),  # streaming
        (9, 1000, torch.float32, True),  # strided logits, contiguous dlogits
        (8, 4096, torch.bfloat16, False),  # bf16 in, fp32 out (32-byte stores)
    ],
)
def test_ce_rows_dlogits_dtype(m, v, dtype, transposed, dev) -> None:
    """dlogits in its own dtype: the same values as the oracle's, rounded once."""
    logits, t = _case(m, v, dtype, dev, seed=3, ignore_every=4, transposed=transposed, scale=3.0)
    out = torch.float32 if dtype == torch.bfloat16 else torch.bfloat16
    loss, lse, dl = ce_rows(logits, t, write_dlogits=True, z_loss_coeff=0.01, dlogits_dtype=out)
    l_ref, lse_ref, dl_ref = OK.ce_rows(logits, t, z_loss_coeff=0.01)
    torch.testing.assert_close(loss.cpu().double(), l_ref, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(lse.cpu().double(), lse_ref, rtol=1e-4, atol=1e-4)
    assert dl.dtype == out and dl.is_contiguous() and dl.shape == (m, v)
    tol = 1e-5 if out == torch.float32 else 1e-2
    torch.testing.assert_close(dl.cpu().double(), dl_ref, rtol=tol, atol=tol)
    if out == torch.bfloat16:  # one rounding of the fp32 value
        same, _, dl32 = ce_rows(logits, t, write_dlogits=True, z_loss_coeff=0.01)
        assert torch.equal(dl, dl32.to(torch.bfloat16)) and torch.equal(same, loss)


def test_ce_rows_cfg4_chunk(dev) -> None:
    """One materialised cfg4 vocab chunk: [16384, 8192] bf16 logits, 1% ignored.

    256 sampled rows against the fp64 oracle; every row: dlogits rows of a
    valid target sum to ~0 (softmax - onehot) and ignored rows are all zero.
    """
    torch.manual_seed(0)
    m, v = 16384, 8192
    logits = (torch.randn(m, v, device=dev) * 2.0).to(torch.bfloat16)
    t = torch.randint(0, v, (m,), device=dev)
    t[torch.rand(m, device=dev) < 0.01] = -100
    loss, lse, dl = ce_rows(logits, t, write_dlogits=True)
    rows = torch.randperm(m, generator=torch.Generator().manual_seed(1))[:256].to(dev)
    l_ref, lse_ref, dl_ref = OK.ce_rows(logits[rows], t[rows])
    torch.testing.assert_close(loss[rows].cpu().double(), l_ref, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(dl[rows].cpu().double(), dl_ref, rtol=1e-2, atol=1e-2)
    sums = dl.float().sum(dim=1)
    assert float(sums.abs().max()) < 5e-2
    ign = t == -100
    assert float(dl[ign].float().abs().sum()) == 0.0


def test_ce_rows_bad_target_is_nan(dev) -> None:
    logits = torch.randn(2, 10, device=dev)
    loss, _, _ = ce_rows(logits, torch.tensor([3, 10], device=dev), write_dlogits=False)
    assert torch.isfinite(loss[0]) and torch.isnan(loss[1])
