"""GPU parity: model inputs of packs built on the device (``pb_pack_tensors``).

Bit-exact against the oracle restatement of dataset.py:33-76 for uint16,
uint32 and int64 token stores, packed and padded packs, empty packs,
one-token documents, a pack filled to the last slot, a pack with hundreds of
documents and a batch of many packs; invalid tables raise ValueError on the
host (the reference raises it for an overflowing pack).  The static-buffer
builder is checked through a captured HIP graph replayed on new tables.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import data as OD
from packbalance_amd.data.device_packs import (
    DeviceTokenStore,
    PackBuilder,
    build_pack_batch,
    segment_table,
)

pytestmark = pytest.mark.gpu

KEYS = ("input_ids", "labels", "position_ids", "doc_ids")


def _random_packs(rng, n_packs, seq_len, n_tokens, max_doc, full=False):
    packs = []
    for _ in range(n_packs):
        segs, used = [], 0
        while True:
            n = int(rng.integers(1, max_doc + 1))
            if used + n > seq_len:
                if full and used < seq_len:
                    n = seq_len - used
                else:
                    break
            segs.append((int(rng.integers(0, n_tokens - n + 1)), n))
            used += n
            if used == seq_len:
                break
        packs.append(segs)
    return packs


def _check(store_np, packs, seq_len, dev, rows=0, pad=0):
    store = DeviceTokenStore(store_np, dev)
    got = build_pack_batch(store, packs, seq_len, rows=rows, pad_token_id=pad)
    want = OD.pack_tensors(store_np, packs, seq_len, rows=rows, pad_token_id=pad)
    for k in KEYS:
        np.testing.assert_array_equal(got[k].cpu().numpy(), want[k], err_msg=k)


@pytest.mark.parametrize("dtype", [np.uint16, np.uint32, np.int64])
def test_packed_batches_match_oracle(dtype, dev) -> None:
    rng = np.random.default_rng(0)
    hi = np.iinfo(np.uint16).max if dtype == np.uint16 else 128256
    tokens = rng.integers(0, hi, size=20000).astype(dtype)
    packs = _random_packs(rng, 4, 2048, len(tokens), 900)
    packs += [[]]                                       # empty pack: all padding
    packs += [[(5, 1), (17, 1), (3, 2)]]                # one-token documents
    packs += _random_packs(rng, 2, 2048, len(tokens), 700, full=True)  # filled to the last slot
    packs += [[(int(s), 4) for s in rng.integers(0, 19990, size=512)]]  # 512 documents
    _check(tokens, packs, 2048, dev, pad=3)


def test_many_packs_and_short_sequences(dev) -> None:
    rng = np.random.default_rng(1)
    tokens = rng.integers(0, 512, size=4000).astype(np.uint32)
    packs = _random_packs(rng, 300, 256, len(tokens), 60)
    _check(tokens, packs, 256, dev)
    _check(tokens, _random_packs(rng, 3, 100, len(tokens), 30), 100, dev)  # seq_len % 8 != 0


def test_padded_packs_match_oracle(dev) -> None:
    rng = np.random.default_rng(2)
    tokens = rng.integers(0, 32000, size=5000).astype(np.uint32)
    rows, seq = 4, 64
    packs = [[(int(rng.integers(0, 4900)), int(rng.integers(1, seq + 1))) for _ in range(r)]
             for r in (4, 3, 1, 0)]
    _check(tokens, packs, seq, dev, rows=rows, pad=9)


def test_invalid_tables_raise(dev) -> None:
    tokens = np.arange(100, dtype=np.uint32)
    store = DeviceTokenStore(tokens, dev)
    with pytest.raises(ValueError):  # overflows seq_len (dataset.py:63-64)
        build_pack_batch(store, [[(0, 40), (40, 30)]], 64)
    with pytest.raises(ValueError):  # outside the store
        build_pack_batch(store, [[(90, 20)]], 64)
    with pytest.raises(ValueError):  # more rows than the padded pack has
        build_pack_batch(store, [[(0, 5)] * 3], 16, rows=2)
    with pytest.raises(ValueError):  # empty document
        build_pack_batch(store, [[(0, 0)]], 16)
    with pytest.raises(TypeError):
        DeviceTokenStore(np.arange(10, dtype=np.float32), dev)


def test_builder_in_a_captured_graph(dev) -> None:
    """PackBuilder: capture launch() once, then replay it on new tables loaded between
    replays (with unrelated eager work in between); every replay matches the oracle."""
    rng = np.random.default_rng(4)
    tokens = rng.integers(0, 32000, size=30000).astype(np.uint32)
    store = DeviceTokenStore(tokens, dev)
    b = PackBuilder(store, 4, 2048)
    steps = [_random_packs(rng, 4, 2048, len(tokens), 800) for _ in range(4)]
    b.load(steps[0])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        b.launch()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        b.launch()
    for packs in steps[1:] + steps[:1]:
        b.load(packs)
        g.replay()
        noise = torch.randn(1 << 16, device=dev).sum()
        torch.cuda.synchronize()
        del noise
        want = OD.pack_tensors(tokens, packs, 2048)
        for k in KEYS:
            np.testing.assert_array_equal(b.outputs[k].cpu().numpy(), want[k], err_msg=k)
        assert b.useful_tokens == sum(n for _, n in (s for p in packs for s in p))
    assert segment_table(steps[0], 2048, len(tokens)).n_packs == 4
