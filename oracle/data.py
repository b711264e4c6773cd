"""CPU restatement of the reference's pack tensors (test oracle).

``pack_tensors`` follows ``packbalance/data/dataset.py:33-76``
(``PackedDataset.__getitem__``) for a batch of packs, each a list of
(start, length) segments of a token array: packed packs place their segments
back to back; padded packs (rows > 0) put segment i in row i of a
rows x seq_len sequence and give the whole row document id i.
Pinned in ``tests/test_oracle.py`` by hand-computed packs and by the
invariants the reference's own tests check (``tests/test_dataset.py:17-59``).
"""

from __future__ import annotations

import numpy as np


def pack_tensors(tokens: np.ndarray, packs, seq_len: int, *, rows: int = 0,
                 pad_token_id: int = 0) -> dict[str, np.ndarray]:
    total = rows * seq_len if rows else seq_len
    n = len(packs)
    out = {
        "input_ids": np.full((n, total), pad_token_id, dtype=np.int64),
        "labels": np.full((n, total), -100, dtype=np.int64),
        "position_ids": np.zeros((n, total), dtype=np.int64),
        "doc_ids": np.full((n, total), -1, dtype=np.int64),
    }
    for p, segs in enumerate(packs):
        offset = 0
        for seg_id, (start, length) in enumerate(segs):
            toks = np.asarray(tokens[start:start + length], dtype=np.int64)
            base = seg_id * seq_len if rows else offset
            out["input_ids"][p, base:base + length] = toks
            if length > 1:
                out["labels"][p, base:base + length - 1] = toks[1:]
            out["position_ids"][p, base:base + length] = np.arange(length)
            if rows:
                out["doc_ids"][p, base:base + seq_len] = seg_id
            else:
                out["doc_ids"][p, base:base + length] = seg_id
            offset += length
        if not rows and offset > seq_len:
            raise ValueError(f"pack {p} overflows seq_len: {offset}")
    return out
