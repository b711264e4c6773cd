"""Model inputs of packs built on the device from a token store in HBM.

The reference builds ``input_ids``, ``labels``, ``position_ids`` and
``doc_ids`` per pack on the host (``packbalance/data/dataset.py:33-76``,
``PackedDataset.__getitem__``) from its memory-mapped token store
(``data/store.py:12-56``) and copies them to the device every micro-batch.
Here the store is loaded into HBM once (``DeviceTokenStore``; 288 GB holds
the whole corpus of any run this targets), the host sends only the step's
segment table -- (start, length) per document, a few KB -- and
``pb_pack_tensors`` writes all four tensors for every pack of the step in one
launch.  The semantics are the reference's: tokens, next-token labels with
-100 on each document's last token, positions restarting at 0 per document,
the segment index as document id; pad_token_id / -100 / 0 / -1 elsewhere;
``rows > 0`` gives the padded form (one document per ``seq_len`` row, the
whole row one document).  Invalid tables raise ``ValueError`` on the host, as
the reference does for a pack that overflows ``seq_len``.

``PackBuilder`` keeps the table and outputs in static device buffers, so a
training step captured in a HIP graph can rebuild its inputs for each new
step from a host-side table copy.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from packbalance_amd import _native as N

MAX_SEGMENTS_PER_PACK = 4096

_ELEM = {np.dtype(np.uint16): 2, np.dtype(np.uint32): 4, np.dtype(np.int64): 8}


class DeviceTokenStore:
    """A token store (``tokens.bin`` of uint16/uint32/int64, plus the per-document
    offsets and lengths) resident in device memory."""

    def __init__(self, tokens: np.ndarray, device, doc_offsets=None, doc_lengths=None) -> None:
        t = np.ascontiguousarray(tokens)
        if t.dtype not in _ELEM:
            raise TypeError(f"token store dtype {t.dtype} is not uint16, uint32 or int64")
        self.elem = _ELEM[t.dtype]
        self.num_tokens = int(t.shape[0])
        self.device = torch.device(device)
        raw = torch.from_numpy(t.view(np.uint8)) if t.size else torch.zeros(16, dtype=torch.uint8)
        self.data = raw.to(self.device)
        self.doc_offsets = None if doc_offsets is None else np.asarray(doc_offsets, dtype=np.int64)
        self.doc_lengths = None if doc_lengths is None else np.asarray(doc_lengths, dtype=np.int64)

    @classmethod
    def open(cls, data_dir: str | Path, device) -> "DeviceTokenStore":
        """The reference's on-disk format (``data/prepare.py:20-56``, ``store.py:21-43``)."""
        data_dir = Path(data_dir)
        meta = json.loads((data_dir / "meta.json").read_text(encoding="utf-8"))
        tokens = np.fromfile(data_dir / "tokens.bin", dtype=np.dtype(meta.get("dtype", "uint32")))
        offsets = np.load(data_dir / "doc_offsets.npy")  # allow_pickle stays False
        lengths = np.load(data_dir / "doc_lengths.npy")
        if len(offsets) != len(lengths):
            raise ValueError("doc_offsets.npy and doc_lengths.npy disagree")
        if len(tokens) != int(meta["num_tokens"]):
            raise ValueError(f"tokens.bin has {len(tokens)} tokens, meta says {meta['num_tokens']}")
        return cls(tokens, device, offsets, lengths)


def _segments(pack) -> list[tuple[int, int]]:
    """(start, length) pairs of a pack: a list of pairs, or an object with
    ``.segments`` whose items have ``.start`` / ``.length`` (the reference's Pack)."""
    segs = getattr(pack, "segments", pack)
    out = []
    for s in segs:
        if hasattr(s, "start"):
            out.append((int(s.start), int(s.length)))
        else:
            out.append((int(s[0]), int(s[1])))
    return out


@dataclass
class SegmentTable:
    seg_start: np.ndarray  # int64 [n_segments]
    seg_len: np.ndarray    # int64 [n_segments]
    pack_seg: np.ndarray   # int64 [n_packs + 1], CSR offsets into the segment arrays
    max_segs: int

    @property
    def n_packs(self) -> int:
        return len(self.pack_seg) - 1


def segment_table(packs, seq_len: int, num_tokens: int, rows: int = 0) -> SegmentTable:
    """Validate packs against the store and the sequence shape (the reference raises
    ValueError when a pack overflows ``seq_len``, dataset.py:63-64)."""
    starts, lens, csr = [], [], [0]
    max_segs = 0
    for i, pack in enumerate(packs):
        segs = _segments(pack)
        if len(segs) > MAX_SEGMENTS_PER_PACK:
            raise ValueError(f"pack {i} has {len(segs)} segments (max {MAX_SEGMENTS_PER_PACK})")
        if rows and len(segs) > rows:
            raise ValueError(f"padded pack {i} has {len(segs)} segments for {rows} rows")
        used = 0
        for start, length in segs:
            if length < 1 or start < 0 or start + length > num_tokens:
                raise ValueError(f"pack {i}: segment ({start}, {length}) is outside the store "
                                 f"of {num_tokens} tokens")
            if rows and length > seq_len:
                raise ValueError(f"pack {i}: a {length}-token row overflows seq_len {seq_len}")
            used += length
            starts.append(start)
            lens.append(length)
        if not rows and used > seq_len:
            raise ValueError(f"pack {i} overflows seq_len: {used}")
        csr.append(len(starts))
        max_segs = max(max_segs, len(segs))
    return SegmentTable(np.asarray(starts, dtype=np.int64), np.asarray(lens, dtype=np.int64),
                        np.asarray(csr, dtype=np.int64), max_segs)


def _launch(store: DeviceTokenStore, starts, lens, csr, n_packs, max_segs, seq_len, rows, pad,
            out: dict) -> None:
    N.call("pb_pack_tensors", store.data.data_ptr(), store.elem, store.num_tokens,
           starts.data_ptr(), lens.data_ptr(), csr.data_ptr(), n_packs, max_segs, seq_len, rows,
           int(pad), out["input_ids"].data_ptr(), out["labels"].data_ptr(),
           out["position_ids"].data_ptr(), out["doc_ids"].data_ptr(), N.stream_ptr(out["doc_ids"]))


def _outputs(n_packs: int, total: int, device) -> dict:
    return {k: torch.empty((n_packs, total), dtype=torch.int64, device=device)
            for k in ("input_ids", "labels", "position_ids", "doc_ids")}


def build_pack_batch(store: DeviceTokenStore, packs, seq_len: int, *, rows: int = 0,
                     pad_token_id: int = 0) -> dict:
    """input_ids, labels, position_ids, doc_ids: int64 [n_packs, seq_len] (or
    [n_packs, rows * seq_len] for padded packs) on the store's device."""
    N.require_device(store.data, op="build_pack_batch")
    tab = segment_table(packs, seq_len, store.num_tokens, rows)
    dev = store.device
    host = torch.from_numpy(np.concatenate([tab.seg_start, tab.seg_len, tab.pack_seg]))
    table = host.pin_memory().to(dev, non_blocking=True)
    ns = len(tab.seg_start)
    out = _outputs(tab.n_packs, rows * seq_len if rows else seq_len, dev)
    _launch(store, table[:ns], table[ns:2 * ns], table[2 * ns:], tab.n_packs, tab.max_segs,
            seq_len, rows, pad_token_id, out)
    return out


class PackBuilder:
    """Static buffers for rebuilding a fixed number of packs every step (graph-safe):
    ``load(packs)`` copies the step's table from pinned host memory (outside any
    captured region; each load stages in a fresh pinned block, which torch's host
    allocator does not reuse before its copy has run, so the host may run steps
    ahead of the device), ``launch()`` writes ``outputs`` (capturable)."""

    def __init__(self, store: DeviceTokenStore, n_packs: int, seq_len: int, *,
                 max_segments: int | None = None, rows: int = 0, pad_token_id: int = 0) -> None:
        N.require_device(store.data, op="PackBuilder")
        self.store, self.n_packs, self.seq_len, self.rows = store, n_packs, seq_len, rows
        self.pad = pad_token_id
        cap = max_segments or n_packs * (rows or seq_len)
        self.cap = int(cap)
        dev = store.device
        # [starts (cap) | lengths (cap) | pack offsets (n_packs + 1) | useful tokens (1)]
        self._table = torch.zeros(2 * self.cap + n_packs + 2, dtype=torch.int64, device=dev)
        self.useful_count = self._table[-1]  # device int64: the step's document tokens
        self.outputs = _outputs(n_packs, rows * seq_len if rows else seq_len, dev)
        # The kernel bounds each pack's segment count by this (its LDS offsets);
        # a captured launch keeps it, so it is the builder's maximum, not a step's.
        self.max_segs = rows if rows else MAX_SEGMENTS_PER_PACK
        self.useful_tokens = 0

    def load(self, packs) -> None:
        if len(packs) != self.n_packs:
            raise ValueError(f"expected {self.n_packs} packs, got {len(packs)}")
        tab = segment_table(packs, self.seq_len, self.store.num_tokens, self.rows)
        ns = len(tab.seg_start)
        if ns > self.cap:
            raise ValueError(f"{ns} segments exceed the builder's capacity {self.cap}")
        h = np.zeros(self._table.numel(), dtype=np.int64)
        h[:ns] = tab.seg_start
        h[self.cap:self.cap + ns] = tab.seg_len
        h[2 * self.cap:2 * self.cap + self.n_packs + 1] = tab.pack_seg
        self.useful_tokens = int(tab.seg_len.sum())
        h[-1] = self.useful_tokens
        self._table.copy_(torch.from_numpy(h).pin_memory(), non_blocking=True)

    def launch(self) -> dict:
        t = self._table
        _launch(self.store, t[:self.cap], t[self.cap:2 * self.cap], t[2 * self.cap:-1],
                self.n_packs, self.max_segs, self.seq_len, self.rows, self.pad, self.outputs)
        return self.outputs
