"""CPU restatement of the document BlockMask tables (test oracle, numpy).

Reference path: ``packbalance/model/attention.py:25-54`` (build_doc_block_mask)
calls torch's ``create_block_mask`` with
    mask_mod(q, kv) = doc[q] == doc[kv] and q >= kv        (attention.py:43-44)
and ``BLOCK = min(block_size, max(32, next_pow2(S)))``      (attention.py:37-41).
torch (``torch/nn/attention/flex_attention.py``) then
  * materialises the dense [B, H, S, S] mask                 (create_mask, :1093-1141)
  * pads it with False to a multiple of BLOCK, sums every block,
    FULL = sum == BLOCK^2, PARTIAL = 0 < sum < BLOCK^2        (:979-1022)
  * orders each row by argsort(descending, stable)           (_dense_to_ordered, :429-436)
  * derives q-major tables by transposing the dense class    (_transpose_ordered, :439-441)

Two independent restatements live here:
  ``tables_dense``  -- the brute-force route above (dense mask, block sums);
  ``tables_closed`` -- a closed form per tile that never builds the mask:
      kv-block > q-block              -> EMPTY (causality)
      kv-block == q-block             -> PARTIAL if any position < S (the
                                          diagonal is allowed, q < kv is not),
                                          FULL only for BLOCK == 1
      kv-block <  q-block             -> FULL if every position < S and one
                                          document covers both blocks; EMPTY if
                                          the two blocks share no document;
                                          else PARTIAL.
``tables_dense`` is pinned against torch's create_block_mask through the
golden fixtures in tests/golden; the two restatements are pinned against each
other on random layouts.
"""

from __future__ import annotations

import numpy as np

EMPTY, PARTIAL, FULL = 0, 1, 2

TABLE_NAMES = (
    "kv_num_blocks",
    "kv_indices",
    "full_kv_num_blocks",
    "full_kv_indices",
    "q_num_blocks",
    "q_indices",
    "full_q_num_blocks",
    "full_q_indices",
)


def doc_block_size(seq_len: int, block_size: int = 128) -> int:
    """BLOCK clamp of reference ``model/attention.py:40-41``."""
    power_of_two = 1 << max(0, seq_len - 1).bit_length()
    return min(block_size, max(32, power_of_two))


def classify_dense(doc: np.ndarray, block: int) -> np.ndarray:
    """[nq, nkv] tile classes by materialising the mask (torch's route)."""
    doc = np.asarray(doc, dtype=np.int64)
    s = doc.shape[0]
    q = np.arange(s)[:, None]
    kv = np.arange(s)[None, :]
    mask = (doc[:, None] == doc[None, :]) & (q >= kv)
    nblk = -(-s // block)
    pad = nblk * block - s
    mask = np.pad(mask, ((0, pad), (0, pad)), constant_values=False)
    sums = mask.reshape(nblk, block, nblk, block).sum(axis=(1, 3))
    cls = np.where(sums == block * block, FULL, np.where(sums > 0, PARTIAL, EMPTY))
    return cls.astype(np.uint8)


def classify_closed(doc: np.ndarray, qblock: int, kvblock: int | None = None) -> np.ndarray:
    """[nq, nkv] tile classes from per-block document sets (no dense mask).

    Supports distinct q / kv tile sizes (used by the attention planner check).
    """
    kvblock = qblock if kvblock is None else kvblock
    doc = np.asarray(doc, dtype=np.int64)
    s = doc.shape[0]
    nq = -(-s // qblock)
    nk = -(-s // kvblock)
    cls = np.zeros((nq, nk), dtype=np.uint8)
    qsets = [np.unique(doc[i * qblock : min(s, (i + 1) * qblock)]) for i in range(nq)]
    ksets = [np.unique(doc[j * kvblock : min(s, (j + 1) * kvblock)]) for j in range(nk)]
    for i in range(nq):
        q0, q1 = i * qblock, (i + 1) * qblock - 1  # token range of the q tile
        for j in range(nk):
            k0, k1 = j * kvblock, (j + 1) * kvblock - 1
            if k0 > q1:
                continue  # every kv after every q
            in_range = q1 < s and k1 < s
            if k1 <= q0:
                # q >= kv for every pair: only documents matter.
                if in_range and qsets[i].size == 1 and ksets[j].size == 1 and qsets[i][0] == ksets[j][0]:
                    cls[i, j] = FULL
                elif np.intersect1d(qsets[i], ksets[j], assume_unique=True).size:
                    cls[i, j] = PARTIAL
                continue
            # Tiles that straddle the diagonal: some q < kv pairs are masked,
            # so at best PARTIAL.  Non-empty iff some q >= kv share a document.
            qa = np.arange(q0, min(q1, s - 1) + 1)
            ka = np.arange(k0, min(k1, s - 1) + 1)
            if qa.size == 0 or ka.size == 0:
                continue
            ok = (doc[qa][:, None] == doc[ka][None, :]) & (qa[:, None] >= ka[None, :])
            if ok.all() and in_range:
                cls[i, j] = FULL
            elif ok.any():
                cls[i, j] = PARTIAL
    return cls


def _ordered(bits: np.ndarray):
    """num, indices of torch's _dense_to_ordered (argsort descending, stable)."""
    bits = bits.astype(np.int32)
    num = bits.sum(axis=-1).astype(np.int32)
    idx = np.argsort(-bits, axis=-1, kind="stable").astype(np.int32)
    return num, idx


def tables_from_classes(cls: np.ndarray, n_heads: int) -> dict[str, np.ndarray]:
    """The eight BlockMask tables for one pack, shaped [1, H, ...] int32."""
    partial = cls == PARTIAL
    full = cls == FULL
    out = {}
    out["kv_num_blocks"], out["kv_indices"] = _ordered(partial)
    out["full_kv_num_blocks"], out["full_kv_indices"] = _ordered(full)
    out["q_num_blocks"], out["q_indices"] = _ordered(partial.T)
    out["full_q_num_blocks"], out["full_q_indices"] = _ordered(full.T)
    for k, v in out.items():
        out[k] = np.ascontiguousarray(np.broadcast_to(v[None, None], (1, n_heads, *v.shape)))
    return out


def tables_dense(doc: np.ndarray, n_heads: int, block: int) -> dict[str, np.ndarray]:
    return tables_from_classes(classify_dense(doc, block), n_heads)


def tables_closed(doc: np.ndarray, n_heads: int, block: int) -> dict[str, np.ndarray]:
    return tables_from_classes(classify_closed(doc, block), n_heads)


def build_doc_block_tables(doc_ids, n_heads: int, block_size: int = 128) -> tuple[dict, int]:
    """Oracle for ``build_doc_block_mask`` (attention.py:25-54): tables + BLOCK.

    ``doc_ids`` is [S] or [1, S]; raises ValueError for B > 1 like the reference.
    """
    doc = np.asarray(doc_ids)
    if doc.ndim == 2:
        if doc.shape[0] != 1:
            raise ValueError("build_doc_block_mask expects a single packed sequence")
        doc = doc[0]
    block = doc_block_size(doc.shape[0], block_size)
    fn = tables_dense if doc.shape[0] <= 4096 else tables_closed
    return fn(doc, n_heads, block), block
