"""GPU parity: document block tables are bit-exact.

Checked against (a) the golden fixtures produced by torch's
create_block_mask, and (b) the numpy oracle on the benchmark workloads
(cfg1 / cfg2 / cfg3 packs), including B > 1 through ``doc_block_tables``.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import block_mask as OB
from packbalance_amd.data import workloads as W
from packbalance_amd.model.attention import build_doc_block_mask, doc_block_tables

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "block_masks.npz"


def _assert_tables(bm_tables: dict, want: dict, what: str) -> None:
    for name in OB.TABLE_NAMES:
        got = bm_tables[name]
        got = got.cpu().numpy() if isinstance(got, torch.Tensor) else got
        assert got.dtype == np.int32, f"{what}:{name} dtype {got.dtype}"
        np.testing.assert_array_equal(got, want[name], err_msg=f"{what}:{name}")


def test_block_tables_match_torch_golden(dev) -> None:
    z = np.load(GOLDEN)
    for name in z["layouts"]:
        name = str(name)
        doc = torch.from_numpy(z[f"{name}/doc_ids"]).to(dev)
        heads = int(z[f"{name}/heads"])
        bm = build_doc_block_mask(doc[None], heads)
        assert bm.BLOCK_SIZE == (int(z[f"{name}/block"]),) * 2, name
        assert bm.seq_lengths == (doc.numel(), doc.numel())
        _assert_tables({n: getattr(bm, n) for n in OB.TABLE_NAMES},
                       {n: z[f"{name}/{n}"] for n in OB.TABLE_NAMES}, name)


@pytest.mark.parametrize("cfg", ["cfg1", "cfg2", "cfg3"])
def test_block_tables_on_benchmark_packs(cfg, dev) -> None:
    if cfg == "cfg1":
        packs, s, heads = W.cfg1_packs(), 256, 4
    elif cfg == "cfg2":
        packs, s, heads = W.cfg2_steps(2)[1], 2048, 12
    else:
        packs, s, heads = W.cfg3_packs(), 8192, 32
    docs = W.doc_ids_from_lengths(packs, s)
    block = OB.doc_block_size(s)
    # Per pack through the reference entry point (B = 1).
    for b in range(len(packs)):
        bm = build_doc_block_mask(docs[b : b + 1].to(dev), heads)
        want = OB.tables_closed(docs[b].numpy(), heads, block)
        _assert_tables({n: getattr(bm, n) for n in OB.TABLE_NAMES}, want, f"{cfg}[{b}]")
    # All packs at once (B > 1 extension).
    t = doc_block_tables(docs.to(dev), heads, block)
    for b in range(len(packs)):
        want = OB.tables_closed(docs[b].numpy(), heads, block)
        _assert_tables({n: t[n][b : b + 1] for n in OB.TABLE_NAMES}, want, f"{cfg}[B={b}]")


@pytest.mark.parametrize("seed", range(4))
def test_block_tables_random_layouts(seed, dev) -> None:
    rng = np.random.default_rng(100 + seed)
    s = int(rng.integers(1, 3000))
    doc = np.sort(rng.integers(0, max(1, s // 50), s))
    if seed % 2:
        doc = rng.permutation(doc)
    if seed >= 2 and s > 8:
        doc[-int(rng.integers(1, 8)):] = -1
    bm = build_doc_block_mask(torch.from_numpy(doc).to(dev), 3)
    block = bm.BLOCK_SIZE[0]
    want = OB.tables_dense(doc, 3, block)
    _assert_tables({n: getattr(bm, n) for n in OB.TABLE_NAMES}, want, f"seed{seed}")


def test_build_doc_block_mask_rejects_batch(dev) -> None:
    with pytest.raises(ValueError):
        build_doc_block_mask(torch.zeros(2, 64, dtype=torch.long, device=dev), 2)


@pytest.mark.parametrize("q_tile,kv_tile,by_kv", [(128, 64, 0), (64, 128, 1), (64, 64, 0), (64, 64, 1)])
def test_attention_plans_match_oracle(q_tile, kv_tile, by_kv, dev) -> None:
    """pb_attn_plan lists == the closed-form tile classes, ascending, each entry
    tile << 2 | kind: 1 FULL, 2 CAUSAL (a partial tile in which every in-range
    pair with kv <= q shares a document, checked densely per tile), 0 PARTIAL."""
    from packbalance_amd import _native as N

    packs = W.cfg3_packs()[:3] + [[5000, 3000, 192]]
    s = 8192
    doc = W.doc_ids_from_lengths(packs, s).to(dev)
    b = doc.shape[0]
    nq, nk = -(-s // q_tile), -(-s // kv_tile)
    rows, cols = (nk, nq) if by_kv else (nq, nk)
    counts = torch.empty((b, rows), dtype=torch.int32, device=dev)
    lists = torch.full((b, rows, cols), -7, dtype=torch.int32, device=dev)
    ws = torch.empty(b * nq * nk, dtype=torch.uint8, device=dev)
    N.call("pb_attn_plan", doc.data_ptr(), doc.stride(0), b, s, q_tile, kv_tile, by_kv,
           counts.data_ptr(), lists.data_ptr(), ws.data_ptr(), N.stream_ptr(doc))
    counts, lists = counts.cpu().numpy(), lists.cpu().numpy()

    def one_doc(d, qi, kj):  # every in-range pair with kv <= q shares a document
        qa = np.arange(qi * q_tile, min((qi + 1) * q_tile, s))
        ka = np.arange(kj * kv_tile, min((kj + 1) * kv_tile, s))
        causal = qa[:, None] >= ka[None, :]
        return bool(np.all((d[qa][:, None] == d[ka][None, :])[causal]))

    kinds = set()
    for i in range(b):
        d = doc[i].cpu().numpy()
        cls = OB.classify_closed(d, q_tile, kv_tile)
        for r in range(rows):
            want = []
            for c in range(cols):
                qi, kj = (c, r) if by_kv else (r, c)
                k = cls[qi, kj]
                if k == OB.FULL:
                    want.append((c << 2) | 1)
                elif k == OB.PARTIAL:
                    want.append((c << 2) | (2 if one_doc(d, qi, kj) else 0))
            kinds.update(w & 3 for w in want)
            assert counts[i, r] == len(want), (i, r)
            assert lists[i, r, : len(want)].tolist() == want, (i, r)
    assert kinds == {0, 1, 2}
