"""GPU parity: the batched transpose that writes the transposed weight copies.

Bit-exact (element bits are copied) against torch's transpose of the same
strided views: bf16 and fp32, full 64 x 64 tiles on 16-byte aligned rows (the
vector path), ragged edges, and shapes whose rows are not 16-byte multiples
(the element path); then ``FlatParams.transposed`` on a store's grouped
weights, rebuilt after the compute copy changes.
"""

from __future__ import annotations

import pytest
import torch

from packbalance_amd import _native as N
from packbalance_amd.model.flat import FlatParams

pytestmark = pytest.mark.gpu


def _transpose(src_buf, offset, batch, rows, cols, bstride, rstride):
    dst = torch.empty((batch, cols, rows), dtype=src_buf.dtype, device=src_buf.device)
    N.call("pb_transpose_batched", src_buf.data_ptr() + offset * src_buf.element_size(), bstride,
           rstride, dst.data_ptr(), batch, rows, cols, src_buf.element_size(),
           N.stream_ptr(src_buf))
    return dst


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("batch,rows,cols,pad_r,pad_b,offset", [
    (12, 1280, 768, 0, 64, 0),     # qkv-shaped, layers at a padded stride
    (3, 768, 2048, 0, 0, 64),      # down-shaped
    (2, 200, 136, 8, 40, 8),       # ragged edge tiles, padded rows
    (2, 67, 45, 3, 7, 1),          # rows not 16-byte multiples: element path
    (1, 1, 1, 0, 0, 0),
])
def test_transpose_matches_torch(dtype, batch, rows, cols, pad_r, pad_b, offset, dev) -> None:
    rstride = cols + pad_r
    bstride = rows * rstride + pad_b
    buf = torch.randn(offset + batch * bstride, device=dev).to(dtype)
    view = buf.as_strided((batch, rows, cols), (bstride, rstride, 1), offset)
    got = _transpose(buf, offset, batch, rows, cols, bstride, rstride)
    assert torch.equal(got, view.transpose(1, 2).contiguous())


def test_transpose_rejects_bad_strides(dev) -> None:
    buf = torch.zeros(64, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        _transpose(buf, 0, 1, 4, 8, 32, 4)  # row stride < cols
    with pytest.raises(ValueError):
        N.call("pb_transpose_batched", buf.data_ptr(), 32, 8, buf.data_ptr(), 1, 4, 8, 3,
               N.stream_ptr(buf))


def test_flat_transposed_groups(dev) -> None:
    layers = torch.nn.ModuleList()
    for _ in range(3):
        m = torch.nn.Module()
        m.a = torch.nn.Linear(96, 160, bias=False)
        m.b = torch.nn.Linear(96, 32, bias=False)
        m.n = torch.nn.Linear(5, 3)  # unaligned sizes between the groups
        layers.append(m)
    layers = layers.to(dev)
    flat = FlatParams(layers, [[m.a.weight, m.b.weight] for m in layers])
    groups = [[m.a.weight, m.b.weight] for m in layers]
    for _ in range(2):
        flat.refresh(torch.bfloat16)
        t = flat.transposed(groups, torch.bfloat16)
        for i, m in enumerate(layers):
            w = torch.cat([m.a.weight, m.b.weight]).to(torch.bfloat16)
            assert torch.equal(t[i], w.t())
        with torch.no_grad():
            flat.master.mul_(1.5)
