"""Write tests/golden/block_masks.npz: FlexAttention BlockMask tables from torch.

The tables come from PyTorch's own ``torch.nn.attention.flex_attention.
create_block_mask`` (the routine the reference calls at
``packbalance/model/attention.py:46-54``), evaluated on the CPU with the
reference's document mask ``doc[q] == doc[kv] and q >= kv`` (attention.py:43-44)
and its BLOCK clamp (attention.py:40-41).  Nothing from the reference tree is
imported.  Re-run after a PyTorch upgrade:

    python tests/golden/make_block_masks.py
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch
from torch.nn.attention.flex_attention import create_block_mask

OUT = Path(__file__).with_name("block_masks.npz")
NAMES = (
    "kv_num_blocks",
    "kv_indices",
    "full_kv_num_blocks",
    "full_kv_indices",
    "q_num_blocks",
    "q_indices",
    "full_q_num_blocks",
    "full_q_indices",
)


def _block(seq_len: int, block_size: int = 128) -> int:
    power_of_two = 1 << max(0, seq_len - 1).bit_length()
    return min(block_size, max(32, power_of_two))


def _lognormal_pack(rng, seq_len, mu, sigma, lo, pad):
    docs, used, d = [], 0, 0
    limit = seq_len - pad
    while used < limit:
        n = int(np.clip(int(rng.lognormal(mu, sigma)), lo, limit - used))
        docs += [d] * n
        used += n
        d += 1
    return docs + [-1] * pad


def layouts() -> list[tuple[str, list[int], int]]:
    rng = np.random.default_rng(1234)
    L = []
    L.append(("one_doc_256", [0] * 256, 2))  # one document: the plain causal block mask
    L.append(("ref_test_64", [0] * 20 + [1] * 44, 2))  # tests/test_attention.py:211
    L.append(("pad_tail_300", [0] * 100 + [1] * 150 + [-1] * 50, 2))
    L.append(("lognormal_2048", _lognormal_pack(rng, 2048, np.log(200), 1.1, 8, 3), 12))
    L.append(("singletons_512", list(range(512)), 1))
    L.append(("alternating_256", [i % 2 for i in range(256)], 2))
    L.append(("random_sorted_1000", sorted(rng.integers(0, 9, 1000).tolist()), 3))
    L.append(("tiny_33", [0] * 10 + [1] * 23, 1))
    L.append(("tiny_17", [0] * 17, 2))
    L.append(("len_1", [0], 1))
    L.append(("aligned_768", [0] * 256 + [1] * 256 + [2] * 256, 4))
    L.append(("boundaries_at_128", sum(([i] * 128 for i in range(16)), []), 2))
    L.append(("one_doc_4096", [0] * 4096, 1))
    L.append(("lognormal_pad_1500", _lognormal_pack(rng, 1500, np.log(48), 0.8, 4, 77), 4))
    L.append(("scrambled_ids_640", rng.permutation(np.repeat(np.arange(5), 128)).tolist(), 2))
    return L


def tables(doc: list[int], n_heads: int):
    ids = torch.tensor(doc, dtype=torch.int64)
    s = ids.numel()
    block = _block(s)

    def mask_mod(b, h, q_idx, kv_idx):
        return (ids[q_idx] == ids[kv_idx]) & (q_idx >= kv_idx)

    bm = create_block_mask(mask_mod, B=1, H=n_heads, Q_LEN=s, KV_LEN=s, device="cpu",
                           BLOCK_SIZE=block)
    return block, {n: getattr(bm, n).numpy().astype(np.int32) for n in NAMES}


def main() -> None:
    arrays: dict[str, np.ndarray] = {}
    names = []
    for name, doc, heads in layouts():
        block, tabs = tables(doc, heads)
        names.append(name)
        arrays[f"{name}/doc_ids"] = np.asarray(doc, dtype=np.int64)
        arrays[f"{name}/block"] = np.asarray(block, dtype=np.int64)
        arrays[f"{name}/heads"] = np.asarray(heads, dtype=np.int64)
        for k, v in tabs.items():
            arrays[f"{name}/{k}"] = v
    arrays["layouts"] = np.asarray(names)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({len(names)} layouts, torch {torch.__version__})")


if __name__ == "__main__":
    main()
